"""numpy fp32 Qwen2 forward, KV cache and greedy decoding (the oracle's model).

Restates `tools/reference/qwen_ref.py` semantics for arbitrary layer count and
vocabulary (shapes come from the weight arrays):
* RMSNorm x * (1/sqrt(mean(x^2) + 1e-6)) * w                      (qwen_ref.py:75-77)
* RoPE rotate_half, theta 1e6, angles in float64, cos/sin rounded once to the compute
  dtype; column j and j+32 of a head share a frequency            (qwen_ref.py:80-81, :118-127)
* GQA: query head h reads KV head h // 7; scores * 0.125; causal mask;
  max-subtracted softmax                                           (qwen_ref.py:139-167)
* o_proj without bias, residual, SwiGLU MLP g/(1+exp(-g)) * u     (qwen_ref.py:168-177)
* tied lm_head over every embedding row                           (qwen_ref.py:188-194)
* greedy: argmax with first-max tie break; a sampled stop token counts toward max_new,
  ends generation and is not in output_ids                        (qwen_ref.py:196-220)
"""
from __future__ import annotations

import numpy as np

HD = 64
HALF = 32
EPS = 1e-6
THETA = 1_000_000.0
SCALE = 0.125
STOP_IDS = (151645, 151643)


def rmsnorm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return (x * (1.0 / np.sqrt(ms + EPS))) * w


def rotate_half(x: np.ndarray) -> np.ndarray:
    return np.concatenate([-x[..., HALF:], x[..., :HALF]], axis=-1)


def rope_cos_sin(pos: np.ndarray, dtype=np.float32):
    """cos/sin [n, 64] for absolute positions `pos` (float64 angles, one rounding)."""
    inv = 1.0 / THETA ** (np.arange(0, HD, 2, dtype=np.float64) / HD)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang).astype(dtype), np.sin(ang).astype(dtype)


class KV:
    """Per-layer K/V [n_kv, max_len, 64]; `len` valid positions."""

    def __init__(self, layers: int, n_kv: int, max_len: int, dtype=np.float32):
        self.k = [np.zeros((n_kv, max_len, HD), dtype) for _ in range(layers)]
        self.v = [np.zeros((n_kv, max_len, HD), dtype) for _ in range(layers)]
        self.len = 0


class Model:
    """Weights as produced by `oracle.illread.load` (or any object with the same fields)."""

    def __init__(self, w, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        c = lambda a: np.ascontiguousarray(a, dtype=self.dtype)  # noqa: E731
        self.embed = c(w.embed)
        self.norm = c(w.norm)
        self.layers = [type(L)(**{k: c(v) for k, v in vars(L).items()}) for L in w.layers]
        self.n_head = self.layers[0].wq.shape[0] // HD
        self.n_kv = self.layers[0].wk.shape[0] // HD
        self.group = self.n_head // self.n_kv
        self.hidden = self.embed.shape[1]

    def new_cache(self, max_len: int) -> KV:
        return KV(len(self.layers), self.n_kv, max_len, self.dtype)

    def attend(self, q, K, V, allowed):
        """q [n, NH, 64] (post-RoPE), K/V [kv, L, 64], allowed [n, L] bool -> [n, H]."""
        n = q.shape[0]
        qg = q.transpose(1, 0, 2).reshape(self.n_kv, self.group, n, HD)
        s = np.matmul(qg, K[:, None].transpose(0, 1, 3, 2)) * self.dtype.type(SCALE)
        s = np.where(allowed[None, None], s, -np.inf)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p = p / p.sum(axis=-1, keepdims=True)
        o = np.matmul(p, V[:, None])
        return o.reshape(self.n_head, n, HD).transpose(1, 0, 2).reshape(n, self.n_head * HD)

    def layer(self, li, x, cos, sin, write_slots, K_slots, allowed, cache: KV, dbg=None):
        """One decoder layer over rows x [n, H].

        write_slots[i]: cache slot receiving row i's K/V. K_slots: the cache slots the
        attention reads (in virtual-position order); allowed [n, len(K_slots)] masks them.
        """
        L = self.layers[li]
        n = x.shape[0]
        h = rmsnorm(x, L.ln1)
        q = (h @ L.wq.T + L.bq).reshape(n, self.n_head, HD)
        k = (h @ L.wk.T + L.bk).reshape(n, self.n_kv, HD)
        v = (h @ L.wv.T + L.bv).reshape(n, self.n_kv, HD)
        c, s_ = cos[:, None, :], sin[:, None, :]
        q_r = q * c + rotate_half(q) * s_
        k_r = k * c + rotate_half(k) * s_
        cache.k[li][:, write_slots] = k_r.transpose(1, 0, 2)
        cache.v[li][:, write_slots] = v.transpose(1, 0, 2)
        K = cache.k[li][:, K_slots]
        V = cache.v[li][:, K_slots]
        o = self.attend(q_r, K, V, allowed)
        attn_out = o @ L.wo.T
        x_mid = x + attn_out
        h2 = rmsnorm(x_mid, L.ln2)
        g = h2 @ L.wg.T
        u = h2 @ L.wu.T
        with np.errstate(over="ignore"):
            act = (g / (1.0 + np.exp(-g))) * u
        out = x_mid + act @ L.wd.T
        if dbg is not None and li == 0:
            dbg.update(l0_attn_norm=h, l0_q_pre_rope=q, l0_k_pre_rope=k, l0_q=q_r, l0_k=k_r,
                       l0_v=v, l0_attn=o, l0_attn_out=attn_out, l0_resid_mid=x_mid,
                       l0_mlp_norm=h2, l0_mlp_act=act, l0_mlp_out=act @ L.wd.T, l0_resid_out=out)
        return out

    def logits(self, x):
        return rmsnorm(x, self.norm) @ self.embed.T

    def forward(self, ids, cache: KV, all_logits: bool = False, dbg: dict | None = None):
        """New tokens `ids` at positions cache.len.. (qwen_ref.py:129-194)."""
        ids = np.asarray(ids, dtype=np.int64)
        n = ids.shape[0]
        p0 = cache.len
        total = p0 + n
        cos, sin = rope_cos_sin(np.arange(p0, total), self.dtype)
        slots = np.arange(p0, total)
        allowed = np.arange(total)[None, :] <= (p0 + np.arange(n))[:, None]
        x = self.embed[ids]
        if dbg is not None:
            dbg["resid"] = [x[-1].copy()]
        for li in range(len(self.layers)):
            x = self.layer(li, x, cos, sin, slots, np.arange(total), allowed, cache, dbg)
            if dbg is not None:
                dbg["resid"].append(x[-1].copy())
        cache.len = total
        if not all_logits:
            x = x[-1:]
        if dbg is not None:
            dbg["final_norm"] = rmsnorm(x, self.norm)[-1].copy()
        lg = self.logits(x)
        return lg if all_logits else lg[0]

    def greedy(self, ids, max_new: int, stop_ids=STOP_IDS, keep_decode_logits: int = 0) -> dict:
        """qwen_ref.py:196-220 semantics."""
        cache = self.new_cache(len(ids) + max_new + 1)
        lg = self.forward(ids, cache)
        last_logits = lg.copy()
        out, step_logits, decode_logits = [], [lg.copy()], []
        stop = None
        for _ in range(max_new):
            tok = int(np.argmax(lg))
            if tok in stop_ids:
                stop = tok
                break
            out.append(tok)
            if len(out) == max_new:
                break
            lg = self.forward([tok], cache)
            step_logits.append(lg.copy())
            if len(decode_logits) < keep_decode_logits:
                decode_logits.append(lg.copy())
        return dict(output_ids=out, stop_token=stop, last_logits=last_logits,
                    step_logits=step_logits, decode_logits=decode_logits)

    def teacher_forced(self, ids, seq) -> tuple[list[int], list[np.ndarray]]:
        """Argmax and logits at positions n-1 .. n-1+len(seq)-1 while feeding `seq`
        (the `forced_argmax` record of tools/reference/README.md:113-136)."""
        cache = self.new_cache(len(ids) + len(seq) + 1)
        lg = self.forward(ids, cache)
        am, lgs = [int(np.argmax(lg))], [lg]
        for t in seq[:-1]:
            lg = self.forward([t], cache)
            am.append(int(np.argmax(lg)))
            lgs.append(lg)
        return am, lgs
