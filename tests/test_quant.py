"""CPU tests of the converter's quantizers (Convert.swift:252-370): the library's C++
quantizers against the oracle's restatement, bit for bit, and the oracle itself pinned by
what the mathematics fixes (exactly representable groups, constant groups, the codes being
the stored pair's nearest codes, never worse than a plain min/max fit)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import quant as OQ

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "instantllm_amd" / "libillhip.so"
needs_lib = pytest.mark.skipif(not LIB.exists(), reason="libillhip.so not built (run __graft_entry__.build())")


def _matrices():
    rng = np.random.default_rng(7)
    out = {
        "gauss": (0.02 * rng.standard_normal((70, 192))).astype(np.float32),
        "outliers": (0.02 * rng.standard_normal((16, 128))).astype(np.float32),
        "skewed": np.abs(0.05 * rng.standard_normal((9, 64))).astype(np.float32) ** 3,
        "wide": (3.0 * rng.standard_normal((5, 256))).astype(np.float32),
    }
    out["outliers"][3, 5] = 1.5
    out["outliers"][7, 70] = -2.0
    m = (0.02 * rng.standard_normal((130, 64))).astype(np.float32)
    m[2] = 0.25                          # constant group
    m[66, :] = 1e-9 * np.arange(64)      # range 6.3e-8: no candidate has a positive f16 scale
    m[67, :] = 0.0
    out["edge"] = m
    return out


@needs_lib
@pytest.mark.parametrize("name", ["gauss", "outliers", "skewed", "wide", "edge"])
def test_q4_library_equals_oracle(name):
    from instantllm_amd.engine import quantize_q4
    w = _matrices()[name]
    p_lib, sb_lib = quantize_q4(w, threads=3)
    p_ref, sb_ref = OQ.q4_rows(w)
    assert np.array_equal(p_lib, p_ref)
    assert np.array_equal(sb_lib.view(np.uint16), sb_ref.view(np.uint16))


@needs_lib
def test_q4_threads_do_not_change_the_bytes():
    from instantllm_amd.engine import quantize_q4
    w = (0.02 * np.random.default_rng(3).standard_normal((300, 128))).astype(np.float32)
    a = quantize_q4(w, threads=1)
    b = quantize_q4(w, threads=7)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1].view(np.uint16), b[1].view(np.uint16))


@needs_lib
@pytest.mark.parametrize("group", [32, 64])
def test_q8_library_equals_oracle(group):
    from instantllm_amd.engine import quantize_q8
    for w in _matrices().values():
        if w.shape[1] % group:
            continue
        c_lib, s_lib = quantize_q8(w, group, threads=2)
        c_ref, s_ref = OQ.q8_rows(w, group)
        assert np.array_equal(c_lib, c_ref)
        assert np.array_equal(s_lib.view(np.uint16), s_ref.view(np.uint16))


def _deq(packed, sb):
    q = np.empty((packed.shape[0], packed.shape[1] * 2), np.float32)
    q[:, 0::2] = packed & 0xF
    q[:, 1::2] = packed >> 4
    s = np.repeat(sb[..., 0].astype(np.float32), 64, axis=1)
    b = np.repeat(sb[..., 1].astype(np.float32), 64, axis=1)
    return q, s * q + b


def test_oracle_q4_recovers_exactly_representable_groups():
    """w = s*q + b with f16 s, b and codes spanning 0..15: the (0, 0) clip fits it exactly,
    so the quantizer must return zero error."""
    rng = np.random.default_rng(11)
    rows = []
    for _ in range(6):
        s = np.float16(rng.uniform(0.001, 0.01)).astype(np.float32)
        b = np.float16(rng.uniform(-0.05, 0.05)).astype(np.float32)
        q = rng.integers(0, 16, 64)
        q[:2] = [0, 15]
        rows.append((s * q + b).astype(np.float32))
    w = np.stack(rows)
    packed, sb = OQ.q4_rows(w)
    _, deq = _deq(packed, sb)
    assert np.array_equal(deq, w)


def test_oracle_q4_constant_group_and_code_rule():
    w = _matrices()["edge"]
    packed, sb = OQ.q4_rows(w)
    q, deq = _deq(packed, sb)
    assert np.all(q[2] == 0) and float(sb[2, 0, 0]) == 0.0 and float(sb[2, 0, 1]) == np.float16(0.25)
    # a range of 6.3e-8: no candidate has a positive f16 scale, so (0, 0) and the codes of
    # the group before it in its 64-row block (quantizeQ4Raw shares the buffer)
    assert float(sb[66, 0, 0]) == 0.0 and float(sb[66, 0, 1]) == 0.0
    assert np.array_equal(q[66], q[65])
    # codes are the stored pair's nearest codes (clamped), wherever the scale is positive
    for r in range(w.shape[0]):
        s, b = sb[r, 0, 0].astype(np.float32), sb[r, 0, 1].astype(np.float32)
        if s > 0:
            want = np.clip(OQ.round_away((w[r] - b) * (np.float32(1) / s)), 0, 15)
            assert np.array_equal(q[r], want), r


def test_oracle_q4_never_worse_than_plain_minmax():
    """The search includes the unclipped range, so its error (float64) is at most the plain
    min/max affine fit's (f16 scale and minimum, nearest codes), up to float32 rounding."""
    w = _matrices()["gauss"].reshape(-1, 64)
    packed, sb = OQ.q4_rows(w)
    _, deq = _deq(packed, sb)
    err = ((deq.astype(np.float64) - w) ** 2).sum(axis=1)
    mn, mx = w.min(axis=1), w.max(axis=1)
    s = ((mx - mn) / 15).astype(np.float16).astype(np.float64)
    b = mn.astype(np.float16).astype(np.float64)
    qm = np.clip(np.floor((w - b[:, None]) / s[:, None] + 0.5), 0, 15)
    err_mm = (((s[:, None] * qm + b[:, None]) - w) ** 2).sum(axis=1)
    assert np.all(err <= err_mm * (1 + 1e-4) + 1e-12)
    assert np.mean(err) < 0.9 * np.mean(err_mm)   # the search and refit do help


def test_oracle_q8_bound_and_ulp_rule():
    w = _matrices()["outliers"]
    q, s = OQ.q8_rows(w, 32)
    assert np.abs(q.astype(np.int32)).max() <= 127
    sf = s.astype(np.float32)
    amax = np.abs(w.reshape(16, 4, 32)).max(axis=2)
    assert np.all(sf * 127 >= amax)                      # every code fits
    lower = (s.view(np.uint16) - 1).view(np.float16).astype(np.float32)
    assert np.all((lower * 127 < amax) | (sf == 0) | (s.view(np.uint16) == np.float16(amax / 127).view(np.uint16)))


CLIP_FIXTURE = ROOT / "tests" / "golden" / "q4_clip_groups.json"


def _clip_groups():
    import json
    doc = json.loads(CLIP_FIXTURE.read_text())
    groups = list(doc["groups"]) + ([doc["refit"]] if doc["refit"] else [])
    w = np.array([g["w"] for g in groups], np.float32)
    return doc, groups, w


def _answers(q, s, b):
    return [(tuple(int(v) for v in q[i]), int(s.view(np.uint16)[i]), int(b.view(np.uint16)[i]))
            for i in range(len(s))]


def _want(groups):
    return [(tuple(g["codes"]), g["scale_f16_bits"], g["bias_f16_bits"]) for g in groups]


def test_oracle_q4_clip_search_known_answers():
    """Hand-evaluated groups (tests/golden/make_q4_clip_fixtures.py: every candidate of
    Convert.swift:319-366 in float64), one won by each clip pair with a margin, and one whose
    least-squares refit moves (scale, bias) off the clipped fit: the oracle returns each
    group's (codes, f16 scale, f16 bias)."""
    doc, groups, w = _clip_groups()
    clips = (0.0, 0.03, 0.06, 0.1, 0.15)
    assert doc["refit"] is not None and len(doc["groups"]) == 25
    assert {tuple(g["pair"]) for g in doc["groups"]} == {(a, c) for a in clips for c in clips}
    assert (doc["refit"]["scale_f16_bits"], doc["refit"]["bias_f16_bits"]) != \
        (doc["refit"]["unrefit_scale_f16_bits"], doc["refit"]["unrefit_bias_f16_bits"])
    q, s, b = OQ.q4_groups(w)
    assert _answers(q, s, b) == _want(groups)


@pytest.mark.parametrize("change", ["drop", "nudge"])
def test_clip_fixtures_catch_a_wrong_clip_constant(monkeypatch, change):
    """A planted mistake in the oracle's clip set (one constant dropped, or moved by 0.01)
    changes the answer of at least one fixture group, for every constant: the fixtures pin
    all five."""
    _, groups, w = _clip_groups()
    want = _want(groups)
    clips = [float(c) for c in OQ.CLIPS]
    for i in range(len(clips)):
        wrong = clips[:i] + clips[i + 1:] if change == "drop" else clips[:i] + [clips[i] + 0.01] + clips[i + 1:]
        monkeypatch.setattr(OQ, "CLIPS", np.array(wrong, np.float32))
        assert _answers(*OQ.q4_groups(w)) != want, (change, clips[i])


@needs_lib
def test_q4_library_clip_search_known_answers():
    """The library's quantizer on the same groups, one group per row."""
    from instantllm_amd.engine import quantize_q4
    _, groups, w = _clip_groups()
    packed, sb = quantize_q4(w, threads=2)
    q = np.empty((w.shape[0], 64), np.int64)
    q[:, 0::2] = packed & 0xF
    q[:, 1::2] = packed >> 4
    assert _answers(q, sb[:, 0, 0], sb[:, 0, 1]) == _want(groups)
