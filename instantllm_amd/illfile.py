"""The `.ill` v1 model container: writer and header reader.

Format (kept identical to the reference so files are interchangeable;
`Sources/Engine/ModelFile.swift:3-5`, `:62-64`, `:113-144`):

* 16 KiB header: u32 magic 0x314D4C49 ("ILM1"), u32 version 1, u32 weight format
  (0 f16, 1 q8, 2 q4), u32 tensor count, then `count` pairs of u64 (offset, size).
* Tensors follow in id order, each 256-byte aligned; the file is padded to 16 KiB.
* Tensor ids (`ModelFile.swift:47-60`): 0 embed, 1 embed scales, 2 final norm,
  3 + 12*layer + k for the per-layer tensors k (0 attn norm, 1 wqkv, 2 wqkv scales,
  3 qkv bias, 4 wo, 5 wo scales, 6 mlp norm, 7 wgu, 8 wgu scales, 9 wd, 10 wd scales),
  and a last id for the optional 2-bit embedding sketch (absent here: size 0).

The reference fixes 24 layers (292 tensors). This writer takes the layer count as a
parameter so that small test models can be built; with 24 layers the output is
byte-compatible with the reference's `ModelWriter`.

Weight payloads are already in the kernel row order: QKV rows in 32-row rotary blocks
(`Convert.swift:236-244`) and gate/up rows interleaved in fours (`Convert.swift:134-136`).
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass

import numpy as np

MAGIC = 0x314D4C49
VERSION = 1
HEADER_SIZE = 16384
PAGE_SIZE = 16384
ALIGN = 256

FMT_F16, FMT_Q8, FMT_Q4 = 0, 1, 2
FMT_NAMES = {FMT_F16: "f16", FMT_Q8: "q8", FMT_Q4: "q4"}

# per-layer tensor slots
ATTN_NORM, WQKV, WQKV_SB, BQKV, WO, WO_SB, MLP_NORM, WGU, WGU_SB, WD, WD_SB = range(11)
PER_LAYER = 12
EMBED, EMBED_SB, FINAL_NORM = 0, 1, 2

HIDDEN = 896
FF = 4864
HEADS = 14
KV_HEADS = 2
HEAD_DIM = 64
QKV_ROWS = 1152
VOCAB = 151936
LAYERS = 24
ROPE_THETA = 1_000_000.0
RMS_EPS = 1e-6
EOS = (151645, 151643)


def layer_id(layer: int, k: int) -> int:
    return 3 + layer * PER_LAYER + k


def tensor_count(layers: int) -> int:
    return 3 + layers * PER_LAYER + 1


def layers_from_count(count: int) -> int:
    if (count - 4) % PER_LAYER:
        raise ValueError(f"tensor count {count} is not 4 + 12*layers")
    return (count - 4) // PER_LAYER


def qkv_row_order() -> np.ndarray:
    """Stored row i of the QKV matrix = original row order[i] of concat(q, k, v).

    36 blocks of 32 rows; block b belongs to head b//2 (0-13 q, 14-15 k, 16-17 v) and
    holds dims half*16+i (rows 0-15) and 32+half*16+i (rows 16-31), half = b%2, so that
    row i and row i+16 are the two members of a rotary pair
    (`Convert.swift:236-244`).
    """
    order = []
    for b in range(36):
        head, half = divmod(b, 2)
        order += [head * 64 + half * 16 + i for i in range(16)]
        order += [head * 64 + 32 + half * 16 + i for i in range(16)]
    return np.asarray(order, dtype=np.int64)


def gu_row_order(ff: int = FF) -> np.ndarray:
    """Stored row 4b+j of gate||up = original row: gate 2b, gate 2b+1, up 2b, up 2b+1
    (`Convert.swift:134-136`)."""
    order = []
    for b in range(ff // 2):
        order += [2 * b, 2 * b + 1, ff + 2 * b, ff + 2 * b + 1]
    return np.asarray(order, dtype=np.int64)


def write_ill(path: str, fmt: int, tensors: dict[int, bytes | np.ndarray], layers: int = LAYERS) -> int:
    """Write an .ill v1 file. `tensors` maps tensor id -> payload (bytes or array, any
    dtype, written raw little-endian). Missing ids get size 0. Returns the file size."""
    count = tensor_count(layers)
    table = np.zeros(2 * count, dtype="<u8")
    cursor = HEADER_SIZE
    layout = []
    for tid in range(count):
        payload = tensors.get(tid)
        if payload is None:
            continue
        if isinstance(payload, np.ndarray):
            payload = np.ascontiguousarray(payload).tobytes()
        cursor = (cursor + ALIGN - 1) & ~(ALIGN - 1)
        table[2 * tid] = cursor
        table[2 * tid + 1] = len(payload)
        layout.append((cursor, payload))
        cursor += len(payload)
    total = (cursor + PAGE_SIZE - 1) // PAGE_SIZE * PAGE_SIZE
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        head = bytearray(HEADER_SIZE)
        struct.pack_into("<IIII", head, 0, MAGIC, VERSION, fmt, count)
        head[16:16 + table.nbytes] = table.tobytes()
        f.write(head)
        pos = HEADER_SIZE
        for off, payload in layout:
            if off > pos:
                f.write(b"\0" * (off - pos))
            f.write(payload)
            pos = off + len(payload)
        if total > pos:
            f.write(b"\0" * (total - pos))
    os.replace(tmp, path)
    return total


@dataclass
class IllHeader:
    fmt: int
    count: int
    layers: int
    offsets: np.ndarray
    sizes: np.ndarray


def read_header(path: str) -> IllHeader:
    with open(path, "rb") as f:
        head = f.read(HEADER_SIZE)
    if len(head) < HEADER_SIZE:
        raise ValueError(f"{path}: shorter than the header")
    magic, version, fmt, count = struct.unpack_from("<IIII", head, 0)
    if magic != MAGIC:
        raise ValueError(f"{path}: not an instantllm model")
    if version != VERSION:
        raise ValueError(f"{path}: unsupported version {version}")
    if fmt not in FMT_NAMES:
        raise ValueError(f"{path}: unknown weight format {fmt}")
    table = np.frombuffer(head, dtype="<u8", count=2 * count, offset=16)
    return IllHeader(fmt, count, layers_from_count(count), table[0::2].copy(), table[1::2].copy())
