"""Pins the CPU oracle: reference golden vectors, closed forms, brute force, invariants."""
from __future__ import annotations

import hashlib
from types import SimpleNamespace

import numpy as np
import pytest

from instantllm_amd import synth, illfile as F
from oracle import qwen, tree as T, metrics, illread

GOLD_LAYERS, GOLD_VOCAB, GOLD_SEED = 2, 1024, 11


def small_weights(seed=GOLD_SEED, layers=GOLD_LAYERS, vocab=GOLD_VOCAB):
    shape = synth.ModelShape(layers=layers, vocab=vocab)
    L = [SimpleNamespace(**synth.float_layer(seed, l, shape)) for l in range(layers)]
    return SimpleNamespace(embed=synth.float_embed(seed, shape), norm=synth.float_norm(seed, shape), layers=L)


@pytest.fixture(scope="module")
def small_model():
    return qwen.Model(small_weights())


def test_fixture_weights_match_generator(golden_small):
    w = small_weights()
    h = hashlib.sha256()
    for a in [w.embed, w.norm] + [getattr(L, k) for L in w.layers for k in sorted(vars(L))]:
        h.update(np.ascontiguousarray(a, np.float32).tobytes())
    assert h.digest() == golden_small["weights_sha256"].tobytes()


def test_greedy_matches_reference(small_model, golden_small):
    ids = golden_small["input_ids"].tolist()
    r = small_model.greedy(ids, max_new=8, keep_decode_logits=7)
    assert r["output_ids"] == golden_small["output_ids"].tolist()
    assert metrics.rel_l2(r["last_logits"], golden_small["last_logits"]) < 1e-5
    dl = np.stack(r["decode_logits"])
    assert dl.shape == golden_small["decode_logits"].shape
    for a, b in zip(dl, golden_small["decode_logits"]):
        assert metrics.rel_l2(a, b) < 1e-5
    for s, top5 in enumerate(golden_small["step_top5"]):
        assert [t for t, _ in metrics.topk(r["step_logits"][s], 5)] == top5.tolist()


def test_debug_tensors_match_reference(small_model, golden_small):
    dbg: dict = {}
    ids = golden_small["input_ids"].tolist()
    small_model.forward(ids, small_model.new_cache(len(ids)), dbg=dbg)
    np.testing.assert_allclose(np.stack(dbg["resid"]), golden_small["resid"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dbg["final_norm"], golden_small["final_norm"], rtol=1e-5, atol=1e-5)
    for name in ("l0_attn_norm", "l0_q_pre_rope", "l0_k_pre_rope", "l0_q", "l0_k", "l0_v",
                 "l0_attn", "l0_attn_out", "l0_resid_mid", "l0_mlp_norm", "l0_mlp_out", "l0_resid_out"):
        np.testing.assert_allclose(dbg[name], golden_small[name], rtol=1e-4, atol=1e-5, err_msg=name)
    np.testing.assert_allclose(dbg["l0_mlp_act"][-1], golden_small["l0_mlp_act_last"], rtol=1e-4, atol=1e-6)


def test_full_prefill_matches_reference(small_model, golden_small):
    seq = golden_small["full_prefill_seq"].tolist()
    lg = small_model.forward(seq, small_model.new_cache(len(seq)))
    assert metrics.rel_l2(lg, golden_small["full_prefill_logits"]) < 1e-5
    la = small_model.forward(seq, small_model.new_cache(len(seq)), all_logits=True)
    assert metrics.rel_l2(la, golden_small["full_prefill_all_logits"]) < 1e-5


def test_kv_cache_decode_equals_reprefill(small_model, golden_small):
    """qwen_ref.py:267-278 invariant, on the oracle itself."""
    ids = golden_small["input_ids"].tolist()
    r = small_model.greedy(ids, max_new=4, keep_decode_logits=3)
    seq = list(ids)
    for j, dl in enumerate(r["decode_logits"]):
        seq.append(r["output_ids"][j])
        full = small_model.forward(seq, small_model.new_cache(len(seq)))
        assert np.abs(full - dl).max() < 1e-4


# ---- closed forms and float64 brute force on tiny inputs -------------------------------

def test_rmsnorm_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 896)).astype(np.float32)
    y = qwen.rmsnorm(x, np.ones(896, np.float32))
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-5)
    w = rng.standard_normal(896).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(qwen.rmsnorm(x, w), ref, rtol=1e-5, atol=1e-6)


def test_rope_rotates_pairs():
    """RoPE is a rotation of each (j, j+32) pair by pos * theta^(-2j/64)."""
    rng = np.random.default_rng(1)
    v = rng.standard_normal(64)
    pos = 37
    cos, sin = qwen.rope_cos_sin(np.array([pos]), np.float64)
    r = v * cos[0] + qwen.rotate_half(v) * sin[0]
    for j in range(32):
        a = pos * 1e6 ** (-2 * j / 64)
        assert np.isclose(r[j], v[j] * np.cos(a) - v[j + 32] * np.sin(a))
        assert np.isclose(r[j + 32], v[j + 32] * np.cos(a) + v[j] * np.sin(a))
    assert np.isclose(np.linalg.norm(r), np.linalg.norm(v))


def test_attention_brute_force():
    """GQA attention against a float64 loop over heads and positions."""
    rng = np.random.default_rng(2)
    m = SimpleNamespace(n_kv=2, group=7, n_head=14, dtype=np.dtype(np.float64))
    q = rng.standard_normal((3, 14, 64))
    K = rng.standard_normal((2, 5, 64))
    V = rng.standard_normal((2, 5, 64))
    allowed = np.array([[1, 1, 1, 0, 0], [1, 1, 1, 1, 0], [1, 0, 1, 0, 1]], bool)
    got = qwen.Model.attend(m, q, K, V, allowed)
    for i in range(3):
        for h in range(14):
            g = h // 7
            s = [(q[i, h] @ K[g, p]) * 0.125 if allowed[i, p] else -np.inf for p in range(5)]
            mx = max(s)
            e = [np.exp(v - mx) for v in s]
            o = sum(e[p] * V[g, p] for p in range(5)) / sum(e)
            np.testing.assert_allclose(got[i, h * 64:(h + 1) * 64], o, rtol=1e-12, atol=1e-12)
    # a single allowed position returns its value row
    one = np.zeros((1, 5), bool)
    one[0, 3] = True
    got1 = qwen.Model.attend(m, q[:1], K, V, one)
    np.testing.assert_allclose(got1[0, :64], V[0, 3])
    np.testing.assert_allclose(got1[0, 7 * 64:8 * 64], V[1, 3])


def test_argmax_ties_lowest_id():
    lg = np.zeros(100, np.float32)
    lg[[7, 42, 99]] = 3.0
    assert metrics.argmax_lowest(lg) == 7
    assert [t for t, _ in metrics.topk(lg, 3)] == [7, 42, 99]


# ---- tree verify semantics -------------------------------------------------------------

def test_tree_rows_equal_sequential_paths(small_model):
    m = small_model
    rng = np.random.default_rng(3)
    ctx = [int(t) for t in rng.integers(0, GOLD_VOCAB, size=9)]
    tr = T.random_tree(rng, 16, GOLD_VOCAB)
    base = m.new_cache(64)
    m.forward(ctx, base)
    tl = T.tree_logits(m, base, tr)
    tok = tr[T.TR_TOK:T.TR_TOK + 16]
    for p in T.paths(tr):
        c = m.new_cache(64)
        m.forward(ctx, c)
        for r in p:
            lg = m.forward([int(tok[r])], c)
            assert metrics.rel_l2(tl[r], lg) < 1e-5, (p, r)


def test_tree_accept_walk():
    # root 0 -> 1 (tok 5), 0 -> 2 (tok 6), 2 -> 3 (tok 8), 1 -> 4 (tok 9)
    tr = T.make_tree([0, 0, 0, 2, 1], [1, 5, 6, 8, 9])
    assert T.accept(tr, [6, 0, 8, 0, 0]) == [2, 3]
    assert T.accept(tr, [5, 9, 0, 0, 0]) == [1, 4]
    assert T.accept(tr, [7, 0, 0, 0, 0]) == []
    out, stop, path = T.commit_tokens(tr, [6, 0, 8, 4, 0], step=0, maxsteps=10)
    assert out == [6, 8, 4] and not stop and path == [2, 3]
    out, stop, _ = T.commit_tokens(tr, [6, 0, 151645, 4, 0], step=0, maxsteps=10)
    assert out == [6, 151645] and stop
    out, stop, _ = T.commit_tokens(tr, [6, 0, 8, 4, 0], step=8, maxsteps=10)
    assert out == [6, 8] and stop
    assert T.chain_accept([5, 6, 7], [5, 6, 1, 0]) == 2
    anc = tr[T.TR_ANC:T.TR_ANC + 5].tolist()
    assert anc == [1, 0b11, 0b101, 0b1101, 0b10011]
    assert tr[T.TR_DEPTH:T.TR_DEPTH + 5].tolist() == [0, 1, 1, 2, 2]


# ---- .ill format round trips ------------------------------------------------------------

@pytest.mark.parametrize("fmt", [F.FMT_F16, F.FMT_Q8, F.FMT_Q4])
def test_ill_roundtrip(tmp_path, fmt):
    shape = synth.ModelShape(layers=1, vocab=64)
    path = str(tmp_path / f"m{fmt}.ill")
    size = synth.build_model(path, fmt, seed=5, shape=shape, q8_group=32 if fmt == F.FMT_Q8 else 64)
    assert size % 16384 == 0
    hdr = F.read_header(path)
    assert hdr.fmt == fmt and hdr.layers == 1
    assert all(o % 256 == 0 for o, s in zip(hdr.offsets, hdr.sizes) if s)
    got = illread.load(path)
    ref = synth.float_layer(5, 0, shape)
    emb = synth.float_embed(5, shape)
    if fmt == F.FMT_F16:
        # f16 stores the generator's values exactly: row orders must be undone exactly
        for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
            np.testing.assert_array_equal(getattr(got.layers[0], k), ref[k], err_msg=k)
        np.testing.assert_array_equal(got.embed, emb)
    else:
        tol = 0.02 * (1.0 if fmt == F.FMT_Q4 else 0.1)
        for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
            assert np.abs(getattr(got.layers[0], k) - ref[k]).max() < tol, k
    for k in ("bq", "bk", "bv", "ln1", "ln2"):
        np.testing.assert_array_equal(getattr(got.layers[0], k), ref[k], err_msg=k)


def test_q4_dequant_closed_form():
    """w = s*q + m with q = low nibble for even columns, high nibble for odd."""
    rng = np.random.default_rng(4)
    w = (0.02 * rng.standard_normal((3, 128))).astype(np.float32)
    packed, sb = synth.quantize_q4(w)
    q = np.empty((3, 128), np.int64)
    q[:, 0::2] = packed & 0xF
    q[:, 1::2] = packed >> 4
    for r in range(3):
        for c in range(128):
            s, mn = float(sb[r, c // 64, 0]), float(sb[r, c // 64, 1])
            assert abs(np.float32(s) * q[r, c] + np.float32(mn) - w[r, c]) <= abs(s) * 0.5 + 1e-3
    codes, sc = synth.quantize_q8(w, 32)
    assert np.abs(codes).max() <= 127
    deq = codes.astype(np.float32).reshape(3, 4, 32) * sc.astype(np.float32)[..., None]
    assert np.abs(deq.reshape(3, 128) - w).max() <= sc.astype(np.float32).max() * 0.5 + 1e-7


def test_tree_buffer_builder_matches_oracle():
    """The package's tree-buffer builder (bench inputs) encodes trees as the oracle does."""
    from instantllm_amd import synth
    for seed in range(20):
        a = synth.random_tree(np.random.default_rng(seed), 16, 151936)
        b = T.random_tree(np.random.default_rng(seed), 16, 151936)
        assert np.array_equal(a, b)
    with pytest.raises(ValueError):
        synth.tree_buffer([0, 1], [5, 6])   # row 1's parent must be an earlier row
