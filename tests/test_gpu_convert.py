"""GPU test of converted checkpoints: a BF16 safetensors checkpoint converted to q4 and q8
(group 32, the reference converter's layout) runs on the engine, and its logits follow the
oracle's forward over the same file (per-step relative L2 <= 1e-2, the config-0 bound)."""
from __future__ import annotations

import numpy as np
import pytest

from instantllm_amd import convert, synth
from oracle import illread, metrics, qwen

from hf_ckpt import checkpoint_tensors, write_checkpoint

pytestmark = pytest.mark.gpu
VOCAB = 2048


@pytest.mark.parametrize("fmt", ["q4", "q8"])
def test_converted_checkpoint_runs(tmp_path, fmt):
    from instantllm_amd.engine import Engine
    d = tmp_path / "hf"
    d.mkdir()
    write_checkpoint(str(d), checkpoint_tensors(5, synth.ModelShape(layers=2, vocab=VOCAB)))
    path = str(tmp_path / f"m_{fmt}.ill")
    convert.convert(str(d), path, fmt, log=lambda *_: None)
    m = qwen.Model(illread.load(path))
    e = Engine(path, max_context=512, max_pass=16, max_steps=64)
    try:
        prompt = [int(t) for t in np.random.default_rng(1).integers(0, VOCAB, 24)]
        e.set_state(pos=0, n=len(prompt), maxsteps=32, eos=(-5, -5))
        e.prefill(prompt, write_logits=True)
        cache = m.new_cache(128)
        ref = m.forward(prompt, cache)
        worst = metrics.rel_l2(e.read_logits(0), ref)
        for s in range(8):
            tok = int(e.out_tokens()[s])
            e.decode_step(write_logits=True)
            ref = m.forward([tok], cache)
            worst = max(worst, metrics.rel_l2(e.read_logits(0), ref))
        print(f"{fmt}: worst per-step rel L2 {worst:.2e}", flush=True)
        assert worst <= 1e-2
    finally:
        e.close()
