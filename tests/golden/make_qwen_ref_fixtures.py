"""Write golden vectors from the reference's own numpy model (run in the build container).

The reference keeps no golden data in its tree (`tools/reference/golden/` is
gitignored) and its loader reads a real bf16 checkpoint that is not available offline.
What pins the oracle's forward composition and greedy semantics is therefore the
reference forward itself, run here on small seeded weights:

* `tools/reference/qwen_ref.py` is imported from /root/reference (read-only), a
  `Qwen2Ref` is built without `__init__` (no checkpoint) and its weight attributes
  (qwen_ref.py:99-119) are assigned from `instantllm_amd.synth` tensors: 2 layers at the
  real widths (896 / 14 q heads / 2 KV heads / 64 / 4864) and a 1024-row vocabulary;
* `greedy` (qwen_ref.py:196-220) with debug dumps (:223-240) and decode logits, and a
  full re-prefill `forward` over the same tokens (the check of :267-278) are recorded.

Only inputs and outputs are stored (`qwen_ref_small.npz`), never reference code. The
reference is not needed at test time.

Usage: python tests/golden/make_qwen_ref_fixtures.py [/root/reference]
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from instantllm_amd import synth  # noqa: E402

SEED = 11
LAYERS = 2
VOCAB = 1024
N_PROMPT = 12
MAX_NEW = 8


def weights_digest(model) -> str:
    h = hashlib.sha256()
    for a in [model.embed, model.norm] + [getattr(L, k) for L in model.layers for k in sorted(vars(L))]:
        h.update(np.ascontiguousarray(a, np.float32).tobytes())
    return h.hexdigest()


def synth_weights():
    shape = synth.ModelShape(layers=LAYERS, vocab=VOCAB)
    layers = [SimpleNamespace(**synth.float_layer(SEED, l, shape)) for l in range(LAYERS)]
    return SimpleNamespace(embed=synth.float_embed(SEED, shape), norm=synth.float_norm(SEED, shape), layers=layers)


def main() -> int:
    ref_root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(ref_root / "tools" / "reference"))
    sys.dont_write_bytecode = True
    import qwen_ref  # noqa: E402  (the reference module, imported read-only)

    w = synth_weights()
    m = object.__new__(qwen_ref.Qwen2Ref)
    m.dtype = np.dtype(np.float32)
    m.embed = np.ascontiguousarray(w.embed, np.float32)
    m.norm = np.ascontiguousarray(w.norm, np.float32)
    m.layers = [SimpleNamespace(**{k: np.ascontiguousarray(v, np.float32) for k, v in vars(L).items()}) for L in w.layers]
    m.inv_freq = 1.0 / qwen_ref.ROPE_THETA ** (np.arange(0, qwen_ref.HEAD_DIM, 2, dtype=np.float64) / qwen_ref.HEAD_DIM)

    rng = np.random.default_rng([SEED, 99])
    ids = [int(t) for t in rng.integers(0, VOCAB, size=N_PROMPT)]
    dbg: dict = {}
    r = m.greedy(ids, max_new=MAX_NEW, keep_decode_logits=MAX_NEW - 1, dbg=dbg)
    out = r["output_ids"]
    # KV-cache consistency (qwen_ref.py:267-278): full prefill over ids + out[:3]
    seq = ids + out[:3]
    full = m.forward(seq, m.new_cache(len(seq)))
    full_all = m.forward(seq, m.new_cache(len(seq)), all_logits=True)

    arrays = dict(
        seed=np.int64(SEED), layers=np.int64(LAYERS), vocab=np.int64(VOCAB),
        weights_sha256=np.frombuffer(bytes.fromhex(weights_digest(w)), np.uint8),
        input_ids=np.asarray(ids, np.int64), output_ids=np.asarray(out, np.int64),
        last_logits=np.asarray(r["last_logits"], np.float32),
        decode_logits=np.stack(r["decode_logits"]).astype(np.float32),
        step_top5=np.asarray([[t for t, _ in s] for s in r["step_top5"]], np.int64),
        full_prefill_seq=np.asarray(seq, np.int64),
        full_prefill_logits=np.asarray(full, np.float32),
        full_prefill_all_logits=np.asarray(full_all, np.float32),
        resid=np.stack(dbg["resid"]).astype(np.float32),
        final_norm=np.asarray(dbg["final_norm"], np.float32),
    )
    for name in ("l0_attn_norm", "l0_q_pre_rope", "l0_k_pre_rope", "l0_q", "l0_k", "l0_v",
                 "l0_attn", "l0_attn_out", "l0_resid_mid", "l0_mlp_norm", "l0_mlp_out", "l0_resid_out"):
        arrays[name] = np.asarray(dbg[name], np.float32)
    arrays["l0_mlp_act_last"] = np.asarray(dbg["l0_mlp_act"][-1], np.float32)
    np.savez_compressed(HERE / "qwen_ref_small.npz", **arrays)
    print("wrote", HERE / "qwen_ref_small.npz", "output_ids", out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
