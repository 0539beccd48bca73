"""Independent `.ill` v1 reader for the oracle: dequantized fp32 weights, HF layout.

Restates the reference's format rules, not the package writer:
* header and tensor table: `Sources/Engine/ModelFile.swift:62-105`;
* q4: byte j of a row holds column 2j (low nibble) and 2j+1 (high nibble); per 64
  columns an f16 (scale, min) pair; w = scale*q + min (`Shaders.swift:118-126`);
* q8: int8 codes, one f16 scale per group (32 in the reference, `Shaders.swift:110-116`;
  the group size is derived from the scale tensor's size), w = scale*q;
* f16: plain half matrix (`Shaders.swift:106-108`);
* QKV stored in 32-row rotary blocks (`Convert.swift:236-244`), gate/up interleaved in
  fours (`Convert.swift:134-136`); both are undone here.
"""
from __future__ import annotations

import struct
from types import SimpleNamespace

import numpy as np

H, FF, NH, NKV, HD = 896, 4864, 14, 2, 64


def _table(buf: memoryview):
    magic, version, fmt, count = struct.unpack_from("<IIII", buf, 0)
    assert magic == 0x314D4C49 and version == 1, "not an ILM1 v1 file"
    t = np.frombuffer(buf, dtype="<u8", count=2 * count, offset=16)
    return fmt, count, t[0::2], t[1::2]


def _mat(buf, fmt, off, size, sboff, sbsize, rows, cols) -> np.ndarray:
    off, size, sboff, sbsize = int(off), int(size), int(sboff), int(sbsize)
    if fmt == 0:
        assert size == rows * cols * 2
        return np.frombuffer(buf, "<f2", rows * cols, off).astype(np.float32).reshape(rows, cols)
    if fmt == 1:
        assert size == rows * cols
        q = np.frombuffer(buf, np.int8, rows * cols, off).astype(np.float32).reshape(rows, cols)
        ngroups = sbsize // 2 // rows
        group = cols // ngroups
        s = np.frombuffer(buf, "<f2", rows * ngroups, sboff).astype(np.float32).reshape(rows, ngroups)
        return (q.reshape(rows, ngroups, group) * s[..., None]).reshape(rows, cols)
    assert fmt == 2 and size == rows * cols // 2
    b = np.frombuffer(buf, np.uint8, rows * cols // 2, off).reshape(rows, cols // 2)
    sb = np.frombuffer(buf, "<f2", rows * cols // 64 * 2, sboff).reshape(rows, cols // 64, 2)
    return dequant_q4(b, sb)


def dequant_q4(codes: np.ndarray, sb: np.ndarray) -> np.ndarray:
    """q4 affine group-64: codes [rows][K/2] (low nibble = even column), sb [rows][K/64][2]
    f16 (scale, min); w = scale * q + min (Shaders.swift:114-126, Convert.swift:67-88)."""
    rows, half = codes.shape
    cols = 2 * half
    q = np.empty((rows, cols), np.float32)
    q[:, 0::2] = codes & 0xF
    q[:, 1::2] = codes >> 4
    s = np.asarray(sb).astype(np.float32).reshape(rows, cols // 64, 2)
    w = q.reshape(rows, cols // 64, 64) * s[..., 0:1] + s[..., 1:2]
    return w.reshape(rows, cols).astype(np.float32)


def _qkv_order():
    o = []
    for b in range(36):
        head, half = divmod(b, 2)
        o += [head * 64 + half * 16 + i for i in range(16)]
        o += [head * 64 + 32 + half * 16 + i for i in range(16)]
    return np.asarray(o)


def _gu_order(ff):
    o = []
    for b in range(ff // 2):
        o += [2 * b, 2 * b + 1, ff + 2 * b, ff + 2 * b + 1]
    return np.asarray(o)


def load(path: str) -> SimpleNamespace:
    """Read an `.ill` file into fp32 arrays: embed [V, H], norm [H] and per layer
    ln1, ln2, wq, bq, wk, bk, wv, bv, wo, wg, wu, wd (HF shapes)."""
    with open(path, "rb") as f:
        data = f.read()
    buf = memoryview(data)
    fmt, count, off, size = _table(buf)
    layers = (count - 4) // 12
    V = int(size[0] * 2 // H) if fmt == 2 else int(size[0] // (H * (2 if fmt == 0 else 1)))
    m = SimpleNamespace(fmt=fmt, layers=[])
    m.embed = _mat(buf, fmt, off[0], size[0], off[1], size[1], V, H)
    m.norm = np.frombuffer(buf, "<f4", H, int(off[2])).copy()
    qinv = np.argsort(_qkv_order())
    ginv = np.argsort(_gu_order(FF))
    for l in range(layers):
        b = 3 + 12 * l
        f32 = lambda k, n: np.frombuffer(buf, "<f4", n, int(off[b + k])).copy()  # noqa: E731
        mat = lambda k, r, c: _mat(buf, fmt, int(off[b + k]), int(size[b + k]),  # noqa: E731
                                   int(off[b + k + 1]), int(size[b + k + 1]), r, c)
        qkv = mat(1, 1152, H)[qinv]
        bias = f32(3, 1152)[qinv]
        gu = mat(7, 2 * FF, H)[ginv]
        m.layers.append(SimpleNamespace(
            ln1=f32(0, H), ln2=f32(6, H),
            wq=qkv[:896], wk=qkv[896:1024], wv=qkv[1024:],
            bq=bias[:896], bk=bias[896:1024], bv=bias[1024:],
            wo=mat(4, H, H), wg=gu[:FF], wu=gu[FF:], wd=mat(9, H, FF),
        ))
    return m
