"""CPU restatement of the reference converter's quantizers (test infrastructure only).

* `q4_rows`: Converter.quantizeQ4Raw + quantGroup (`Sources/Engine/Convert.swift:286-370`):
  per 64-column group, clipped ranges [mn + a*range, mx - c*range] for a, c in
  {0, .03, .06, .1, .15} (`Convert.swift:319`), one least-squares refit of (scale, bias) on
  the clipped fit's codes (`:336-351`), both rounded to f16, codes re-derived with the
  stored values, lowest squared error kept (strict `<`, so the first candidate on ties,
  `:353-366`); a group with range < 1e-12 gets zero codes, scale 0, bias f16(mn)
  (`:325-328`). The code buffer is shared by the groups of a 64-row block (`:300-306`).
* `q8_rows`: Converter.quantizeQ8 (`Convert.swift:252-282`).

Arithmetic is float32 in the reference's order (Swift `Float`); sums run over the 64
values one after the other, as the reference's loop does; `.rounded()` is half away from
zero; `Float16(x)` rounds to nearest even. Vectorized over groups, sequential over the 64
values of a group, so it is slow but exact on small inputs.
"""
from __future__ import annotations

import numpy as np

CLIPS = np.array([0.0, 0.03, 0.06, 0.1, 0.15], np.float32)
f32 = np.float32


def round_away(x: np.ndarray) -> np.ndarray:
    """Swift `.rounded()` on float32 values (half away from zero), exact via float64."""
    x64 = np.asarray(x, np.float64)
    return (np.sign(x64) * np.floor(np.abs(x64) + 0.5)).astype(np.float32)


def _codes(w, b, inv):
    """min(15, max(0, round((w - b) * inv))) for w [G, 64], b/inv [G] (rows whose inv is
    not finite give NaN codes; no candidate of such a row is ever taken)."""
    with np.errstate(invalid="ignore", over="ignore"):
        t = ((w - b[:, None]).astype(np.float32) * inv[:, None]).astype(np.float32)
        return np.minimum(f32(15), np.maximum(f32(0), round_away(t)))


def q4_groups(w: np.ndarray):
    """Groups w [G, 64] float32 -> (codes [G, 64] u8 or -1 where the reference keeps the
    previous group's codes, scale f16 [G], bias f16 [G])."""
    w = np.ascontiguousarray(w, np.float32)
    G = w.shape[0]
    mn = w.min(axis=1)
    mx = w.max(axis=1)
    rng_ = (mx - mn).astype(np.float32)
    best_err = np.full(G, np.inf, np.float32)
    best_s = np.zeros(G, np.float16)
    best_b = np.zeros(G, np.float16)
    best_q = np.full((G, 64), -1, np.int16)   # -1: no candidate chosen
    flat = rng_ < f32(1e-12)
    for a in CLIPS:
        for c in CLIPS:
            lo = (mn + (a * rng_).astype(np.float32)).astype(np.float32)
            hi = (mx - (c * rng_).astype(np.float32)).astype(np.float32)
            ok = (hi > lo) & ~flat
            s = ((hi - lo).astype(np.float32) / f32(15)).astype(np.float32)
            b = lo.copy()
            active = ok.copy()
            for it in range(2):
                with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
                    inv = (f32(1) / s).astype(np.float32)
                v = _codes(w, b, inv)
                sq = np.zeros(G, np.float32)
                sw = np.zeros(G, np.float32)
                sqq = np.zeros(G, np.float32)
                sqw = np.zeros(G, np.float32)
                for i in range(64):
                    vi, wi = v[:, i], w[:, i]
                    sq = (sq + vi).astype(np.float32)
                    sw = (sw + wi).astype(np.float32)
                    sqq = (sqq + (vi * vi).astype(np.float32)).astype(np.float32)
                    sqw = (sqw + (vi * wi).astype(np.float32)).astype(np.float32)
                if it == 1:
                    break
                den = ((f32(64) * sqq).astype(np.float32) - (sq * sq).astype(np.float32)).astype(np.float32)
                refit = active & (den > 0)
                with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
                    s2 = (((f32(64) * sqw).astype(np.float32) - (sq * sw).astype(np.float32)).astype(np.float32)
                          / den).astype(np.float32)
                refit &= s2 > 0
                b2 = ((sw - (s2 * sq).astype(np.float32)).astype(np.float32) / f32(64)).astype(np.float32)
                s = np.where(refit, s2, s).astype(np.float32)
                b = np.where(refit, b2, b).astype(np.float32)
            with np.errstate(over="ignore"):
                sh = s.astype(np.float16)
                bh = b.astype(np.float16)
            sf = sh.astype(np.float32)
            bf = bh.astype(np.float32)
            cand = ok & (sf > 0)
            with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
                inv = (f32(1) / sf).astype(np.float32)
            v = _codes(w, bf, inv)
            err = np.zeros(G, np.float32)
            for i in range(64):
                d = ((sf * v[:, i]).astype(np.float32) + bf).astype(np.float32)
                d = (d - w[:, i]).astype(np.float32)
                err = (err + (d * d).astype(np.float32)).astype(np.float32)
            take = cand & (err < best_err)
            best_err = np.where(take, err, best_err)
            best_s = np.where(take, sh, best_s)
            best_b = np.where(take, bh, best_b)
            best_q = np.where(take[:, None], np.nan_to_num(v).astype(np.int16), best_q)
    best_s = np.where(flat, np.float16(0), best_s)
    best_b = np.where(flat, mn.astype(np.float16), best_b)
    best_q = np.where(flat[:, None], 0, best_q)
    return best_q, best_s, best_b


def q4_rows(w: np.ndarray):
    """Matrix w [rows, cols] -> (packed u8 [rows, cols/2], sb f16 [rows, cols/64, 2]) as
    quantizeQ4Raw writes them (codes kept from the previous group of the same 64-row block
    where no candidate had a positive f16 scale)."""
    rows, cols = w.shape
    gpr = cols // 64
    q, s, b = q4_groups(w.reshape(rows * gpr, 64))
    q = q.reshape(rows, gpr, 64)
    prev = np.zeros(64, np.int16)
    for r in range(rows):
        if r % 64 == 0:
            prev = np.zeros(64, np.int16)
        for g in range(gpr):
            if q[r, g, 0] < 0:
                q[r, g] = prev
            prev = q[r, g].copy()
    q = q.reshape(rows, cols).astype(np.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    sb = np.stack([s.reshape(rows, gpr), b.reshape(rows, gpr)], axis=-1)
    return packed, sb


def q8_rows(w: np.ndarray, group: int = 32):
    """quantizeQ8: codes i8 [rows, cols], scales f16 [rows, cols/group]."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    g = w.reshape(rows, cols // group, group)
    amax = np.abs(g).max(axis=2)
    sh = (amax / f32(127)).astype(np.float32).astype(np.float16)
    low = (sh.astype(np.float32) * f32(127)).astype(np.float32) < amax
    sh = np.where(low, (sh.view(np.uint16) + 1).view(np.float16), sh)
    s = sh.astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(s > 0, (f32(1) / np.where(s > 0, s, f32(1))).astype(np.float32), f32(0)).astype(np.float32)
    t = (g * inv[..., None]).astype(np.float32)
    q = np.maximum(f32(-127), np.minimum(f32(127), round_away(t))).astype(np.int8)
    return q.reshape(rows, cols), sh
