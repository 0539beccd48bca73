"""Hugging Face checkpoint -> `.ill` converter (Converter.convert, Convert.swift:91-214).

Reads a Qwen2.5-0.5B-shaped checkpoint (`model.safetensors`, or shards listed in
`model.safetensors.index.json`; BF16 tensors) and writes an `.ill` v1 file the engine
loads:

* embedding (also the tied lm_head) and per layer the QKV (q, k, v rows concatenated and
  stored in 32-row rotary blocks), O, gate||up (rows interleaved in fours) and down
  matrices, quantized to q4 (affine, group 64: the reference quantizer `quantGroup`,
  Convert.swift:321-370), q8 (symmetric, group 32 by default: `quantizeQ8`, :254-282) or
  stored as f16;
* RMSNorm weights, the final norm and the QKV bias (same row order) as f32.

An optional quant file (`--quant`, Convert.swift:96-122) supplies q4 codes for a matrix
as `<name>.q` (U8 [rows][cols/2]), `<name>.scale` and `<name>.bias` (F16 [rows][cols/64]),
and may override the unquantized vectors (norms, biases; any float dtype).

Not converted: the reference's `q4a` format and its 2-bit embedding sketch (this engine
runs neither); a separate `lm_head.weight` (the model ties it to the embedding, and so
does the file format).

Usage: python -m instantllm_amd.convert HF_DIR OUT.ill --format q4|q8|f16 [--quant FILE]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import struct
import sys

import numpy as np

from . import illfile as F

_DT = {"BF16": ("<u2", 2), "F16": ("<f2", 2), "F32": ("<f4", 4), "U8": ("u1", 1), "I8": ("i1", 1)}


class SafeTensors:
    """A safetensors file, memory-mapped: 8-byte header length, JSON header, raw data."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            self.header = json.loads(f.read(n))
        self.data_start = 8 + n
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        self.entries = {k: v for k, v in self.header.items() if k != "__metadata__"}

    def has(self, name: str) -> bool:
        return name in self.entries

    def raw(self, name: str) -> tuple[np.ndarray, str, list[int]]:
        if name not in self.entries:
            raise KeyError(f"missing tensor {name}")
        e = self.entries[name]
        dt, size = _DT[e["dtype"]]
        a, b = e["data_offsets"]
        buf = self.mm[self.data_start + a:self.data_start + b]
        return buf.view(dt), e["dtype"], list(e["shape"])

    def floats(self, name: str) -> np.ndarray:
        """Any float tensor as float32 (BF16 widened exactly), in its shape."""
        v, dt, shape = self.raw(name)
        if dt == "BF16":
            out = (v.astype(np.uint32) << 16).view(np.float32)
        elif dt in ("F16", "F32"):
            out = v.astype(np.float32)
        else:
            raise ValueError(f"{name}: expected a float tensor, got {dt}")
        return out.reshape(shape)


class Checkpoint:
    """One safetensors file or the shards of an index."""

    def __init__(self, hf_dir: str):
        single = os.path.join(hf_dir, "model.safetensors")
        index = os.path.join(hf_dir, "model.safetensors.index.json")
        self.files: dict[str, SafeTensors] = {}
        self.where: dict[str, str] = {}
        if os.path.exists(single):
            st = SafeTensors(single)
            self.files[single] = st
            self.where = {k: single for k in st.entries}
        elif os.path.exists(index):
            with open(index) as f:
                wm = json.load(f)["weight_map"]
            for name, fn in wm.items():
                p = os.path.join(hf_dir, fn)
                if p not in self.files:
                    self.files[p] = SafeTensors(p)
                self.where[name] = p
        else:
            raise FileNotFoundError(f"{hf_dir}: no model.safetensors or model.safetensors.index.json")

    def has(self, name: str) -> bool:
        return name in self.where

    def floats(self, name: str) -> np.ndarray:
        if name not in self.where:
            raise KeyError(f"missing tensor {name}")
        return self.files[self.where[name]].floats(name)

    def layers(self) -> int:
        ids = {int(m.group(1)) for k in self.where for m in [re.match(r"model\.layers\.(\d+)\.", k)] if m}
        n = max(ids) + 1 if ids else 0
        if ids != set(range(n)):
            raise ValueError("checkpoint layers are not numbered 0..n-1")
        return n


def _q4_bytes(w: np.ndarray) -> tuple[bytes, bytes]:
    from .engine import quantize_q4
    p, sb = quantize_q4(np.ascontiguousarray(w, np.float32))
    return p.tobytes(), sb.astype("<f2").tobytes()


def _q8_bytes(w: np.ndarray, group: int) -> tuple[bytes, bytes]:
    from .engine import quantize_q8
    q, s = quantize_q8(np.ascontiguousarray(w, np.float32), group)
    return q.tobytes(), s.astype("<f2").tobytes()


def convert(hf_dir: str, output: str, fmt: str = "q4", quant_file: str | None = None, q8_group: int = 32,
            log=print) -> int:
    """Convert the checkpoint in `hf_dir` to `output`; returns the file size."""
    fmt_id = {"f16": F.FMT_F16, "q8": F.FMT_Q8, "q4": F.FMT_Q4}[fmt]
    ck = Checkpoint(hf_dir)
    qf = SafeTensors(quant_file) if quant_file else None
    if qf is not None and fmt_id != F.FMT_Q4:
        raise ValueError("quant files hold q4 codes; use --format q4")
    H, FF = F.HIDDEN, F.FF

    def vec(name):
        if qf is not None and qf.has(name):
            return qf.floats(name).reshape(-1)
        return ck.floats(name).reshape(-1)

    def q4_override(name):
        """(packed, sb) bytes from the quant file, or None."""
        if qf is None or not qf.has(name + ".q"):
            return None
        codes, dt, shape = qf.raw(name + ".q")
        sc, sdt, _ = qf.raw(name + ".scale")
        bi, bdt, _ = qf.raw(name + ".bias")
        if dt != "U8" or sdt != "F16" or bdt != "F16":
            raise ValueError(f"{name}: bad quant dtypes")
        rows = shape[0]
        sb = np.stack([sc.reshape(rows, -1), bi.reshape(rows, -1)], axis=-1)
        return np.ascontiguousarray(codes).reshape(rows, -1), sb.reshape(rows, -1)

    def matrix(names, order=None):
        """The concatenated rows of `names` (in `order`) as (weights, scales) payloads."""
        if fmt_id == F.FMT_Q4:
            parts = []
            for n in names:
                o = q4_override(n)
                if o is None:
                    w = ck.floats(n)
                    p, sb = _q4_bytes(w)
                    rows = w.shape[0]
                    o = (np.frombuffer(p, np.uint8).reshape(rows, -1), np.frombuffer(sb, "<f2").reshape(rows, -1))
                parts.append(o)
            codes = np.concatenate([p for p, _ in parts])
            sb = np.concatenate([s for _, s in parts])
            if order is not None:
                codes, sb = codes[order], sb[order]
            return np.ascontiguousarray(codes).tobytes(), np.ascontiguousarray(sb).astype("<f2").tobytes()
        w = np.concatenate([ck.floats(n) for n in names])
        if order is not None:
            w = w[order]
        if fmt_id == F.FMT_Q8:
            return _q8_bytes(w, q8_group)
        return w.astype("<f2").tobytes(), b""

    layers = ck.layers()
    emb = ck.floats("model.embed_tokens.weight")
    if emb.shape[1] != H:
        raise ValueError(f"hidden size {emb.shape[1]} (the engine is built for {H})")
    tensors: dict[int, bytes | np.ndarray] = {}
    tensors[F.EMBED], tensors[F.EMBED_SB] = matrix(["model.embed_tokens.weight"])
    tensors[F.FINAL_NORM] = vec("model.norm.weight").astype("<f4")
    log(f"embedding done ({emb.shape[0]} x {emb.shape[1]})")
    del emb
    qo = F.qkv_row_order()
    go = F.gu_row_order(FF)
    for l in range(layers):
        p = f"model.layers.{l}."
        L = lambda k: F.layer_id(l, k)  # noqa: E731
        tensors[L(F.ATTN_NORM)] = vec(p + "input_layernorm.weight").astype("<f4")
        tensors[L(F.MLP_NORM)] = vec(p + "post_attention_layernorm.weight").astype("<f4")
        bias = np.concatenate([vec(p + "self_attn.q_proj.bias"), vec(p + "self_attn.k_proj.bias"),
                               vec(p + "self_attn.v_proj.bias")])
        tensors[L(F.BQKV)] = bias[qo].astype("<f4")
        tensors[L(F.WQKV)], tensors[L(F.WQKV_SB)] = matrix(
            [p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight", p + "self_attn.v_proj.weight"], qo)
        tensors[L(F.WO)], tensors[L(F.WO_SB)] = matrix([p + "self_attn.o_proj.weight"])
        tensors[L(F.WGU)], tensors[L(F.WGU_SB)] = matrix([p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"], go)
        tensors[L(F.WD)], tensors[L(F.WD_SB)] = matrix([p + "mlp.down_proj.weight"])
        log(f"layer {l} done")
    size = F.write_ill(output, fmt_id, tensors, layers)
    log(f"wrote {output} ({size} bytes, {layers} layers, {fmt})")
    return size


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("hf_dir")
    ap.add_argument("output")
    ap.add_argument("--format", default="q4", choices=["q4", "q8", "f16"])
    ap.add_argument("--quant", default=None, help="safetensors file of q4 codes / vector overrides")
    ap.add_argument("--q8-group", type=int, default=32, choices=[32, 64])
    a = ap.parse_args(argv)
    convert(a.hf_dir, a.output, a.format, a.quant, a.q8_group)
    return 0


if __name__ == "__main__":
    sys.exit(main())
