"""Seeded synthetic Qwen2.5-0.5B-shaped models in the `.ill` v1 layout.

There is no network, so every model the engine runs is generated here from a seed with
`numpy.random.default_rng`. Each tensor draws from its own child generator
`default_rng([seed, tensor_key])`, so a model with fewer layers or a smaller vocabulary
holds exactly the same values as the full model in the tensors they share.

Distributions: matrices N(0, 0.02) rounded to f16, QKV biases
N(0, 0.02), RMSNorm weights N(1, 0.1). q4 and q8 models quantize those float weights with
the reference converter's own quantizers (`quantizer="reference"`, the default: the
clipped-range search with a least-squares refit of `Sources/Engine/Convert.swift:286-370`
and the symmetric q8 of `:252-282`, run by libillhip.so's `ill_quantize_q4` /
`ill_quantize_q8`), so the kernels see the code distributions a converted checkpoint has.
`quantizer="minmax"` selects the plain min/max affine q4 (`quantize_q4`) instead. The CPU
oracle consumes the dequantized values either way.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import illfile as F

_LAYER_KEYS = ("ln1", "ln2", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "wg", "wu", "wd")


@dataclass(frozen=True)
class ModelShape:
    layers: int = F.LAYERS
    vocab: int = F.VOCAB
    hidden: int = F.HIDDEN
    ff: int = F.FF
    heads: int = F.HEADS
    kv_heads: int = F.KV_HEADS
    head_dim: int = F.HEAD_DIM


def _key(name: str, layer: int = -1) -> int:
    if layer < 0:
        return {"embed": 0, "norm": 1}[name]
    return 100 + 16 * layer + _LAYER_KEYS.index(name)


def _rng(seed: int, key: int) -> np.random.Generator:
    return np.random.default_rng([seed, key])


def _f16_round(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float16).astype(np.float32)


def gen_tensor(seed: int, name: str, layer: int, shape: tuple[int, ...]) -> np.ndarray:
    """One float32 tensor of the synthetic model in the HF [out, in] layout."""
    g = _rng(seed, _key(name, layer))
    if name in ("ln1", "ln2", "norm"):
        return (1.0 + 0.1 * g.standard_normal(shape, dtype=np.float32)).astype(np.float32)
    if name in ("bq", "bk", "bv"):
        return (0.02 * g.standard_normal(shape, dtype=np.float32)).astype(np.float32)
    return _f16_round(0.02 * g.standard_normal(shape, dtype=np.float32))


def layer_shapes(s: ModelShape) -> dict[str, tuple[int, ...]]:
    H, FFd, hd = s.hidden, s.ff, s.head_dim
    return {
        "ln1": (H,), "ln2": (H,),
        "wq": (s.heads * hd, H), "bq": (s.heads * hd,),
        "wk": (s.kv_heads * hd, H), "bk": (s.kv_heads * hd,),
        "wv": (s.kv_heads * hd, H), "bv": (s.kv_heads * hd,),
        "wo": (H, s.heads * hd),
        "wg": (FFd, H), "wu": (FFd, H), "wd": (H, FFd),
    }


def float_layer(seed: int, layer: int, s: ModelShape = ModelShape()) -> dict[str, np.ndarray]:
    return {k: gen_tensor(seed, k, layer, shp) for k, shp in layer_shapes(s).items()}


def float_embed(seed: int, s: ModelShape = ModelShape()) -> np.ndarray:
    return gen_tensor(seed, "embed", -1, (s.vocab, s.hidden))


def float_embed_chunks(seed: int, s: ModelShape = ModelShape(), rows: int = 8192):
    """The embedding in row chunks: the same values as `float_embed` (one generator,
    drawn in order) without materializing the whole table."""
    g = _rng(seed, _key("embed"))
    for r0 in range(0, s.vocab, rows):
        n = min(rows, s.vocab - r0)
        yield _f16_round(0.02 * g.standard_normal((n, s.hidden), dtype=np.float32))


def float_norm(seed: int, s: ModelShape = ModelShape()) -> np.ndarray:
    return gen_tensor(seed, "norm", -1, (s.hidden,))


# ----------------------------------------------------------------------------------------
# quantizers (format: Shaders.swift:110-126 embed_at; Convert.swift:67-88, :254-282)

def quantize_q4(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Affine group-64 4-bit: w ~ s*q + m, q in 0..15, (s, m) f16 per 64 columns.

    Returns (packed u8 [rows, cols/2] with column 2j in the low nibble of byte j,
    sb f16 [rows, cols/64, 2] holding (scale, min)).
    """
    rows, cols = w.shape
    g = w.reshape(rows, cols // 64, 64).astype(np.float32)
    lo = g.min(axis=2)
    hi = g.max(axis=2)
    s16 = ((hi - lo) / 15.0).astype(np.float16)
    s16 = np.where(s16 == 0, np.float16(6.1e-5), s16)
    m16 = lo.astype(np.float16)
    s = s16.astype(np.float32)[..., None]
    m = m16.astype(np.float32)[..., None]
    q = np.clip(np.rint((g - m) / s), 0, 15).astype(np.uint8).reshape(rows, cols)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    sb = np.stack([s16, m16], axis=-1)
    return packed, sb


def quantize_q8(w: np.ndarray, group: int = 64) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int8 per `group` columns with an f16 scale: w ~ s*q, q in -127..127.
    The scale is the f16 value nearest amax/127, bumped one ulp when it would leave a
    code out of range (the rule of `Convert.swift:254-282`)."""
    rows, cols = w.shape
    g = w.reshape(rows, cols // group, group).astype(np.float32)
    amax = np.abs(g).max(axis=2)
    s16 = (amax / 127.0).astype(np.float16)
    low = s16.astype(np.float32) * 127.0 < amax
    s16 = np.where(low, (s16.view(np.uint16) + 1).view(np.float16), s16)
    s = s16.astype(np.float32)
    inv = np.where(s > 0, 1.0 / np.where(s > 0, s, 1.0), 0.0).astype(np.float32)
    q = np.clip(np.rint(g * inv[..., None]), -127, 127).astype(np.int8).reshape(rows, cols)
    return q, s16


def _emit_matrix(fmt: int, w: np.ndarray, q8_group: int, quantizer: str = "reference") -> tuple[bytes, bytes]:
    if quantizer not in ("reference", "minmax"):
        raise ValueError(f"unknown quantizer {quantizer!r}")
    if fmt == F.FMT_Q4:
        if quantizer == "reference":
            from .engine import quantize_q4 as lib_q4
            p, sb = lib_q4(w)
        else:
            p, sb = quantize_q4(w)
        return p.tobytes(), sb.astype("<f2").tobytes()
    if fmt == F.FMT_Q8:
        if quantizer == "reference":
            from .engine import quantize_q8 as lib_q8
            q, sc = lib_q8(w, q8_group)
        else:
            q, sc = quantize_q8(w, q8_group)
        return q.tobytes(), sc.astype("<f2").tobytes()
    return w.astype("<f2").tobytes(), b""


def build_model(path: str, fmt: int, seed: int, shape: ModelShape = ModelShape(),
                q8_group: int = 64, quantizer: str = "reference") -> int:
    """Generate the seeded model and write it as an `.ill` v1 file. Returns its size."""
    tensors: dict[int, bytes | np.ndarray] = {}
    wparts, sparts = [], []
    for chunk in float_embed_chunks(seed, shape):
        w, sb = _emit_matrix(fmt, chunk, q8_group, quantizer)
        wparts.append(w)
        sparts.append(sb)
    tensors[F.EMBED], tensors[F.EMBED_SB] = b"".join(wparts), b"".join(sparts)
    del wparts, sparts
    tensors[F.FINAL_NORM] = float_norm(seed, shape).astype("<f4")
    qo = F.qkv_row_order()
    go = F.gu_row_order(shape.ff)
    for l in range(shape.layers):
        t = float_layer(seed, l, shape)
        L = lambda k: F.layer_id(l, k)  # noqa: E731
        tensors[L(F.ATTN_NORM)] = t["ln1"].astype("<f4")
        tensors[L(F.MLP_NORM)] = t["ln2"].astype("<f4")
        bias = np.concatenate([t["bq"], t["bk"], t["bv"]])
        tensors[L(F.BQKV)] = bias[qo].astype("<f4")
        qkv = np.concatenate([t["wq"], t["wk"], t["wv"]], axis=0)[qo]
        tensors[L(F.WQKV)], tensors[L(F.WQKV_SB)] = _emit_matrix(fmt, qkv, q8_group, quantizer)
        tensors[L(F.WO)], tensors[L(F.WO_SB)] = _emit_matrix(fmt, t["wo"], q8_group, quantizer)
        gu = np.concatenate([t["wg"], t["wu"]], axis=0)[go]
        tensors[L(F.WGU)], tensors[L(F.WGU_SB)] = _emit_matrix(fmt, gu, q8_group, quantizer)
        tensors[L(F.WD)], tensors[L(F.WD_SB)] = _emit_matrix(fmt, t["wd"], q8_group, quantizer)
    return F.write_ill(path, fmt, tensors, shape.layers)


# ----------------------------------------------------------------------------------------
# config-1 microbench operands: random q4 codes (not a quantized float matrix)

def microbench_q4(seed: int, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """Codes uniform in [0, 15], scale |N(0, 0.01)| f16, min N(0, 0.01) f16."""
    g = np.random.default_rng([seed, rows, cols])
    q = g.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    s = np.abs(0.01 * g.standard_normal((rows, cols // 64), dtype=np.float32)).astype(np.float16)
    m = (0.01 * g.standard_normal((rows, cols // 64), dtype=np.float32)).astype(np.float16)
    return packed, np.stack([s, m], axis=-1)


def microbench_x(seed: int, cols: int, rows: int = 1) -> tuple[np.ndarray, np.ndarray]:
    """x f16 N(0, 1) (returned as float32 values) and gamma N(1, 0.1)."""
    g = np.random.default_rng([seed, 7, cols])
    x = g.standard_normal((rows, cols), dtype=np.float32).astype(np.float16).astype(np.float32)
    gamma = (1.0 + 0.1 * g.standard_normal(cols, dtype=np.float32)).astype(np.float32)
    return x, gamma


def tree_buffer(parent: list[int], tok: list[int]) -> np.ndarray:
    """The 65-int tree buffer of a verify pass, [n, depth[16], parent[16], tok[16], anc[16]]
    (Sources/Engine/Shaders.swift:23-30), from parent indices (parent[0] ignored)."""
    n = len(tok)
    if not (1 <= n <= 16 and len(parent) == n):
        raise ValueError("a tree has 1..16 rows")
    t = np.zeros(65, np.int32)
    t[0] = n
    depth, anc = [0] * n, [1] * n
    for i in range(1, n):
        p = parent[i]
        if not 0 <= p < i:
            raise ValueError(f"parent[{i}] = {p} is not an earlier row")
        depth[i] = depth[p] + 1
        anc[i] = anc[p] | (1 << i)
    t[1:1 + n] = depth
    t[17:17 + n] = [0] + list(parent[1:])
    t[33:33 + n] = tok
    t[49:49 + n] = anc
    return t


def random_tree(rng: np.random.Generator, n: int, vocab: int) -> np.ndarray:
    """Config 3 tree: parent[i] uniform over rows 0..i-1, tokens uniform in [0, vocab)."""
    parent = [0] + [int(rng.integers(0, i)) for i in range(1, n)]
    tok = [int(t) for t in rng.integers(0, vocab, size=n)]
    return tree_buffer(parent, tok)


def cached_model(fmt: int, seed: int, shape: ModelShape = ModelShape(), directory: str | None = None) -> str:
    """Path of the seeded synthetic model, generated once into `directory`
    (default $ILL_MODEL_DIR or /tmp/ill_models)."""
    import os
    d = directory or os.environ.get("ILL_MODEL_DIR", "/tmp/ill_models")
    os.makedirs(d, exist_ok=True)
    tag = "" if shape == ModelShape() else f"_L{shape.layers}_V{shape.vocab}"
    qtag = "_rq" if fmt != F.FMT_F16 else ""   # the reference converter's quantizers
    p = os.path.join(d, f"qwen05b_fmt{fmt}_seed{seed}{tag}{qtag}.ill")
    if not os.path.exists(p):
        tmp = p + f".tmp{os.getpid()}"
        build_model(tmp, fmt, seed, shape=shape)
        os.replace(tmp, p)
    return p
