"""CPU tests of the checkpoint converter (instantllm_amd/convert.py; Converter.convert,
Convert.swift:91-214): a BF16 safetensors checkpoint of the synthetic model converts to an
`.ill` file whose weights, read back by the oracle's independent reader (undoing the row
orders), are the checkpoint's: exactly for f16 (= the f16 rounding of the BF16 values) and
within the quantizers' error for q8 / q4."""
from __future__ import annotations

import numpy as np
import pytest

from instantllm_amd import convert, synth
from oracle import illread

from hf_ckpt import checkpoint_tensors, write_checkpoint, write_safetensors

SHAPE = synth.ModelShape(layers=2, vocab=1024)
MATS = ["wq", "wk", "wv", "wo", "wg", "wu", "wd"]
HF = {"wq": "self_attn.q_proj.weight", "wk": "self_attn.k_proj.weight", "wv": "self_attn.v_proj.weight",
      "wo": "self_attn.o_proj.weight", "wg": "mlp.gate_proj.weight", "wu": "mlp.up_proj.weight",
      "wd": "mlp.down_proj.weight", "bq": "self_attn.q_proj.bias", "bk": "self_attn.k_proj.bias",
      "bv": "self_attn.v_proj.bias", "ln1": "input_layernorm.weight", "ln2": "post_attention_layernorm.weight"}


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("hf")
    t = checkpoint_tensors(3, SHAPE)
    write_checkpoint(str(d), t)
    return str(d), t


def _vectors_equal(m, t):
    np.testing.assert_array_equal(m.norm, t["model.norm.weight"])
    for l, L in enumerate(m.layers):
        for k in ("ln1", "ln2", "bq", "bk", "bv"):
            np.testing.assert_array_equal(getattr(L, k), t[f"model.layers.{l}.{HF[k]}"])


def test_f16_exact_and_row_orders(ckpt, tmp_path):
    d, t = ckpt
    out = str(tmp_path / "m.ill")
    convert.convert(d, out, "f16", log=lambda *_: None)
    m = illread.load(out)
    f16 = lambda a: a.astype(np.float16).astype(np.float32)  # noqa: E731
    np.testing.assert_array_equal(m.embed, f16(t["model.embed_tokens.weight"]))
    _vectors_equal(m, t)
    for l, L in enumerate(m.layers):
        for k in MATS:
            np.testing.assert_array_equal(getattr(L, k), f16(t[f"model.layers.{l}.{HF[k]}"]), err_msg=f"{l} {k}")


def test_q8_group32_within_half_step(ckpt, tmp_path):
    d, t = ckpt
    out = str(tmp_path / "m8.ill")
    convert.convert(d, out, "q8", log=lambda *_: None)
    m = illread.load(out)
    _vectors_equal(m, t)
    for l, L in enumerate(m.layers):
        for k in MATS:
            w = t[f"model.layers.{l}.{HF[k]}"]
            g = w.reshape(w.shape[0], -1, 32)
            step = np.abs(g).max(axis=-1, keepdims=True) / 127
            err = np.abs(getattr(L, k).reshape(g.shape) - g)
            assert (err <= 0.5 * step * 1.01 + 1e-8).all(), (l, k)


def test_q4_sharded_checkpoint(tmp_path):
    """Shards listed in model.safetensors.index.json convert like one file; q4 weights are
    within the affine quantizer's error (a misordered row would be off by ~1.4x)."""
    d1, d2 = tmp_path / "one", tmp_path / "sharded"
    d1.mkdir()
    d2.mkdir()
    t = checkpoint_tensors(3, SHAPE)
    write_checkpoint(str(d1), t)
    write_checkpoint(str(d2), t, shards=3)
    a, b = str(tmp_path / "a.ill"), str(tmp_path / "b.ill")
    convert.convert(str(d1), a, "q4", log=lambda *_: None)
    convert.convert(str(d2), b, "q4", log=lambda *_: None)
    assert open(a, "rb").read() == open(b, "rb").read()
    m = illread.load(a)
    _vectors_equal(m, t)
    for l, L in enumerate(m.layers):
        for k in MATS:
            w = t[f"model.layers.{l}.{HF[k]}"]
            rel = np.linalg.norm(getattr(L, k) - w) / np.linalg.norm(w)
            assert rel < 0.12, (l, k, rel)


def test_quant_file_overrides(ckpt, tmp_path):
    """A quant file's q4 codes and vector overrides are written as given (Convert.swift:96-122)."""
    d, t = ckpt
    rng = np.random.default_rng(0)
    name = "model.layers.1.self_attn.o_proj.weight"
    codes = rng.integers(0, 256, (896, 448), dtype=np.uint8)
    sc = rng.normal(0, 0.01, (896, 14)).astype(np.float16)
    bi = rng.normal(0, 0.01, (896, 14)).astype(np.float16)
    norm = rng.normal(1, 0.1, 896).astype(np.float32)
    qf = str(tmp_path / "quant.safetensors")
    write_safetensors(qf, {name + ".q": (codes, "U8"), name + ".scale": (sc, "F16"), name + ".bias": (bi, "F16"),
                           "model.norm.weight": (norm, "F32")})
    out = str(tmp_path / "mq.ill")
    convert.convert(d, out, "q4", quant_file=qf, log=lambda *_: None)
    m = illread.load(out)
    np.testing.assert_array_equal(m.norm, norm)
    sb = np.stack([sc, bi], axis=-1)
    np.testing.assert_array_equal(m.layers[1].wo, illread.dequant_q4(codes, sb))
    with pytest.raises(ValueError, match="use --format q4"):
        convert.convert(d, str(tmp_path / "x.ill"), "q8", quant_file=qf, log=lambda *_: None)


def test_missing_tensor_and_directory(tmp_path):
    with pytest.raises(FileNotFoundError):
        convert.convert(str(tmp_path), str(tmp_path / "o.ill"), "q4", log=lambda *_: None)
    t = checkpoint_tensors(3, synth.ModelShape(layers=1, vocab=256))
    del t["model.layers.0.mlp.down_proj.weight"]
    write_checkpoint(str(tmp_path), t)
    with pytest.raises(KeyError, match="down_proj"):
        convert.convert(str(tmp_path), str(tmp_path / "o.ill"), "f16", log=lambda *_: None)
