"""GPU parity of the HIP engine against the CPU oracle, through the C ABI.

Small seeded q4 models (2-4 layers, vocabulary 4096, real widths) keep the numpy oracle
fast; the full-size model is covered by size-independent properties in
test_gpu_fullsize.py. Tolerances: per-step logits relative L2
<= 1e-2 against the fp32 oracle, teacher-forced greedy agreement >= 99%, and 1-row vs
16-row logits bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

from instantllm_amd import synth, illfile as F
from oracle import illread, qwen, metrics, tree as T

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-2
VOCAB = 4096


def log(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def q4_small(tmp_path_factory):
    d = tmp_path_factory.mktemp("q4")
    path = str(d / "small_q4.ill")
    synth.build_model(path, F.FMT_Q4, seed=2, shape=synth.ModelShape(layers=3, vocab=VOCAB))
    return path, qwen.Model(illread.load(path))


@pytest.fixture(scope="module")
def engine(q4_small):
    from instantllm_amd.engine import Engine
    log("engine: create small q4 (3 layers, vocab 4096)")
    e = Engine(q4_small[0], max_context=1024, max_pass=16, max_steps=256)
    yield e
    e.close()


def test_prefill_and_decode_logits(engine, q4_small):
    _, m = q4_small
    rng = np.random.default_rng(10)
    prompt = [int(t) for t in rng.integers(0, VOCAB, size=37)]
    log("prefill 37 tokens (3 chunks) + 12 decode steps")
    engine.set_state(pos=0, n=len(prompt), maxsteps=64, eos=(-5, -5))
    engine.prefill(prompt, write_logits=True)
    cache = m.new_cache(128)
    ref = m.forward(prompt, cache)
    lg = engine.read_logits(0)
    assert metrics.rel_l2(lg, ref) <= REL_L2_TOL
    assert int(engine.out_tokens()[0]) == int(np.argmax(lg))   # commit == argmax of the logits
    tok = int(np.argmax(lg))
    for s in range(12):
        engine.decode_step(write_logits=True)
        lg = engine.read_logits(0)
        ref = m.forward([tok], cache)
        assert metrics.rel_l2(lg, ref) <= REL_L2_TOL, s
        nxt = int(engine.out_tokens()[s + 1])
        assert nxt == int(np.argmax(lg)), "commit must pick the lowest-id argmax of the row's logits"
        tok = nxt
    st = engine.get_state()
    assert st["pos"] == len(prompt) + 12 and st["step"] == 13


def test_teacher_forced_agreement(engine, q4_small):
    """Greedy tokens of the GPU vs the oracle's argmax on the same (GPU) sequence."""
    _, m = q4_small
    rng = np.random.default_rng(11)
    prompt = [int(t) for t in rng.integers(0, VOCAB, size=20)]
    log("generate 32 tokens with captured graphs")
    toks = engine.generate(prompt, max_new=32, chunk=8)
    assert len(toks) == 32 or (len(toks) < 32 and engine.get_state()["done"])
    am, lgs = m.teacher_forced(prompt, toks)
    agree, n = metrics.forced_agreement(toks, am)
    assert agree / n >= 0.99, (agree, n)


def test_generate_matches_stepwise(engine):
    """Graph-captured generation == the same steps launched one by one."""
    rng = np.random.default_rng(12)
    prompt = [int(t) for t in rng.integers(0, VOCAB, size=9)]
    a = engine.generate(prompt, max_new=20, chunk=4)
    engine.reset_out_tokens()
    engine.set_state(pos=0, n=len(prompt), maxsteps=20)
    engine.prefill(prompt)
    for _ in range(19):
        engine.decode_step()
    b = [int(t) for t in engine.out_tokens()[:20]]
    stop = next((i for i, t in enumerate(b) if t in (151645, 151643)), None)
    assert a == (b if stop is None else b[:stop])


def _ctx(engine, rng, n):
    ctx = [int(t) for t in rng.integers(0, VOCAB, size=n)]
    engine.reset_out_tokens()
    engine.set_state(pos=0, n=n, maxsteps=200, eos=(-5, -5))
    engine.prefill(ctx)
    return ctx, engine.get_state()


def test_decode_across_a_chunk_end(engine, q4_small):
    """Decode steps at positions 58-67: the chunk holding the new position runs to its
    last slots (pos % 64 in 58-63) and then a new chunk starts."""
    _, m = q4_small
    rng = np.random.default_rng(13)
    prompt = [int(t) for t in rng.integers(0, VOCAB, size=58)]
    engine.reset_out_tokens()
    engine.set_state(pos=0, n=len(prompt), maxsteps=64, eos=(-5, -5))
    engine.prefill(prompt, write_logits=True)
    cache = m.new_cache(128)
    assert metrics.rel_l2(engine.read_logits(0), m.forward(prompt, cache)) <= REL_L2_TOL
    tok = int(engine.out_tokens()[0])
    for s in range(10):
        engine.decode_step(write_logits=True)
        lg = engine.read_logits(0)
        assert metrics.rel_l2(lg, m.forward([tok], cache)) <= REL_L2_TOL, s
        tok = int(engine.out_tokens()[s + 1])


def test_overlong_requests_are_refused(engine):
    """Engine.swift:934: a request that cannot fit in the context is refused before any
    launch; a live state must leave room for a 16-row pass."""
    from instantllm_amd.engine import IllError, ILL_E_ARG
    with pytest.raises(IllError) as ei:
        engine.generate([1] * 100, max_new=engine.max_context - 100)
    assert ei.value.code == ILL_E_ARG
    for bad in (dict(pos=engine.max_context - 8), dict(step=64), dict(step=-1), dict(n=0), dict(n=engine.max_context + 1)):
        kw = dict(pos=0, n=1, maxsteps=64)
        kw.update(bad)
        with pytest.raises(IllError):
            engine.set_state(**kw)
    # a done state is accepted whatever its counters (the host parks a finished request)
    engine.set_state(pos=engine.max_context - 8, n=1, maxsteps=64, done=1)


def test_decode_stops_at_the_context_end(engine):
    """Steps launched past the context early-exit: the commit sets the stop flag once a
    following pass would not fit (pos + 16 > max_context)."""
    rng = np.random.default_rng(14)
    n = engine.max_context - 24
    prompt = [int(t) for t in rng.integers(0, VOCAB, size=n)]
    engine.reset_out_tokens()
    engine.set_state(pos=0, n=n, maxsteps=200, eos=(-5, -5))
    engine.prefill(prompt)
    for _ in range(20):
        engine.decode_step()
    st = engine.get_state()
    # the step at pos = max_context - 16 is the last one that runs
    assert st["done"] == 1 and st["pos"] == engine.max_context - 15, st
    assert st["step"] == 1 + (engine.max_context - 16 - n) + 1


@pytest.mark.parametrize("prefix", [60, 100, 300])
def test_tree_rows_bit_identical_to_sequential_steps(engine, prefix):
    """Config 3 invariant: every tree row's logits equal, bit for bit, the logits of the
    same token decoded as a 1-row step after its ancestors."""
    rng = np.random.default_rng(20 + prefix)
    ctx, st = _ctx(engine, rng, prefix)
    tr = T.random_tree(rng, 16, VOCAB)
    log(f"tree pass at pos {st['pos']}")
    engine.set_state(pos=st["pos"], n=16, maxsteps=200, eos=(-5, -5))
    engine.verify_pass(16, tree=tr, write_logits=True)
    rows = np.stack([engine.read_logits(r) for r in range(16)])
    tok = tr[T.TR_TOK:T.TR_TOK + 16]
    for p in T.paths(tr):
        for k, r in enumerate(p):
            engine.set_state(pos=st["pos"] + k, n=1, maxsteps=200, eos=(-5, -5))
            engine.prefill([int(tok[r])], write_logits=True)
            one = engine.read_logits(0)
            assert np.array_equal(one.view(np.uint32), rows[r].view(np.uint32)), (p, k, r)


@pytest.mark.parametrize("prefix,nrows", [(61, 4), (300, 3), (130, 2)])
def test_small_tree_rows_bit_identical(engine, prefix, nrows):
    """Trees of 3-4 rows run on the 16-row kernel, of 2 rows on the 4-row kernel: still equal
    to 1-row steps bit for bit."""
    rng = np.random.default_rng(25 + prefix)
    ctx, st = _ctx(engine, rng, prefix)
    tr = T.random_tree(rng, nrows, VOCAB)
    engine.set_state(pos=st["pos"], n=nrows, maxsteps=200, eos=(-5, -5))
    engine.verify_pass(nrows, tree=tr, write_logits=True)
    rows = np.stack([engine.read_logits(r) for r in range(nrows)])
    tok = tr[T.TR_TOK:T.TR_TOK + nrows]
    for p in T.paths(tr):
        for k, r in enumerate(p):
            engine.set_state(pos=st["pos"] + k, n=1, maxsteps=200, eos=(-5, -5))
            engine.prefill([int(tok[r])], write_logits=True)
            one = engine.read_logits(0)
            assert np.array_equal(one.view(np.uint32), rows[r].view(np.uint32)), (p, k, r)


def test_tree_logits_match_oracle(engine, q4_small):
    _, m = q4_small
    rng = np.random.default_rng(30)
    ctx, st = _ctx(engine, rng, 70)
    tr = T.random_tree(rng, 16, VOCAB)
    engine.set_state(pos=st["pos"], n=16, maxsteps=200, eos=(-5, -5))
    engine.verify_pass(16, tree=tr, write_logits=True)
    cache = m.new_cache(128)
    m.forward(ctx, cache)
    ref = T.tree_logits(m, cache, tr)
    for r in range(16):
        assert metrics.rel_l2(engine.read_logits(r), ref[r]) <= REL_L2_TOL, r


def test_tree_accept_commit_and_kv_compaction(engine, q4_small):
    """A tree whose drafts follow the model's own argmaxes is accepted along that path;
    the committed tokens, state and compacted K/V match the oracle's sequential decode."""
    _, m = q4_small
    rng = np.random.default_rng(40)
    ctx, st = _ctx(engine, rng, 50)
    pos0 = st["pos"]
    cache = m.new_cache(128)
    m.forward(ctx[:-1], cache)
    root = int(engine.out_tokens()[0])
    # oracle greedy continuation from the committed token
    seq, c2 = [root], m.new_cache(128)
    m.forward(ctx, c2)
    lg = m.forward([root], c2)
    for _ in range(4):
        seq.append(int(np.argmax(lg)))
        lg = m.forward([seq[-1]], c2)
    # tree: root -> 1 (wrong) ; root -> 2 (= seq[1]) -> 3 (wrong), 2 -> 4 (= seq[2]) -> 5 (= seq[3])
    wrong = lambda t: (t + 7) % VOCAB  # noqa: E731
    parent = [0, 0, 0, 2, 2, 4]
    toks = [root, wrong(seq[1]), seq[1], wrong(seq[2]), seq[2], seq[3]]
    tr = T.make_tree(parent, toks)
    engine.reset_out_tokens()
    engine.set_state(pos=pos0, n=6, maxsteps=200, eos=(-5, -5))
    engine.verify_pass(6, tree=tr, write_logits=True)
    g = [int(np.argmax(engine.read_logits(r))) for r in range(6)]
    out, stop, path = T.commit_tokens(tr, g, step=0, maxsteps=200, eos=(-5, -5))
    got = [int(t) for t in engine.out_tokens()[: len(out)]]
    assert got == out
    assert path == [2, 4, 5], (g, seq)
    st2 = engine.get_state()
    assert st2["pos"] == pos0 + len(path) + 1 and st2["accepted"] == len(path) and st2["passes"] == 1
    # after compaction, a decode step continues exactly like sequential decoding
    engine.decode_step(write_logits=True)
    c3 = m.new_cache(128)
    m.forward(ctx, c3)
    for t in [root, seq[1], seq[2], seq[3]]:
        ref = m.forward([t], c3)
    ref = m.forward([out[-1]], c3)
    assert metrics.rel_l2(engine.read_logits(0), ref) <= REL_L2_TOL


def test_chain_pass_commit(engine, q4_small):
    rng = np.random.default_rng(50)
    ctx, st = _ctx(engine, rng, 30)
    root = int(engine.out_tokens()[0])
    engine.reset_out_tokens()
    engine.set_state(pos=st["pos"], n=4, maxsteps=200, eos=(-5, -5))
    drafts = [5, 6, 7]
    engine.verify_pass(4, toks=[root] + drafts, write_logits=True)
    g = [int(np.argmax(engine.read_logits(r))) for r in range(4)]
    m_acc = T.chain_accept(drafts, g)
    got = [int(t) for t in engine.out_tokens()[: m_acc + 1]]
    assert got == g[: m_acc + 1]
    assert engine.get_state()["pos"] == st["pos"] + m_acc + 1


def test_kv_copy_roundtrip(engine):
    rng = np.random.default_rng(60)
    _ctx(engine, rng, 40)
    k, v = engine.kv_copy_out(40)
    assert k.shape == (3, 2, 40, 64) and np.any(k) and np.any(v)
    engine.kv_copy_in(np.zeros_like(k), np.zeros_like(v))
    z = engine.kv_copy_out(40)
    assert not np.any(z[0]) and not np.any(z[1])
    engine.kv_copy_in(k, v)
    k2, v2 = engine.kv_copy_out(40)
    assert np.array_equal(k, k2) and np.array_equal(v, v2)


def test_stop_token_and_maxsteps(engine):
    rng = np.random.default_rng(70)
    prompt = [int(t) for t in rng.integers(0, VOCAB, size=8)]
    engine.reset_out_tokens()
    engine.set_state(pos=0, n=8, maxsteps=3, eos=(-5, -5))
    engine.prefill(prompt)
    for _ in range(5):
        engine.decode_step()
    st = engine.get_state()
    assert st["step"] == 3 and st["done"] == 1
    first = int(engine.out_tokens()[0])
    # making the first generated token a stop id ends the request right there
    engine.reset_out_tokens()
    engine.set_state(pos=0, n=8, maxsteps=30, eos=(first, -5))
    engine.prefill(prompt)
    engine.decode_step()
    st = engine.get_state()
    assert st["done"] == 1 and st["step"] == 1


def test_host_stop_ends_queued_steps(engine):
    """Engine.generate's onToken stop (Engine.swift:1021-1036): the callback stops the
    request after the 5th token of a 32-step graph; the steps still queued leave at once.
    The device advanced by no more than the steps that were already running, and the cached
    prefix is the prompt plus the delivered tokens (a follow-up request over them reuses
    it and continues exactly as a cold greedy run)."""
    e = engine
    prompt = [int(t) for t in np.random.default_rng(77).integers(0, 4096, size=20)]
    e.truncate_cache(0)
    ref = e.generate(prompt, max_new=40, chunk=8)
    seen = []
    e.truncate_cache(0)
    got = e.generate(prompt, max_new=32, chunk=32, on_token=lambda t: (seen.append(t), len(seen) < 5)[1])
    assert got == ref[:5] and seen == ref[:5]
    st = e.get_state()
    # prefill commits token 0 at pos len(prompt); step k commits token k: at most the step in
    # flight when the host stopped, and the one whose commit found the stop word, ran
    assert st["done"] == 1
    assert st["pos"] <= len(prompt) + 4 + 2, st
    assert st["step"] <= 5 + 1, st
    cached, _ = e.prefix_info()
    assert cached == len(prompt) + 4
    # a follow-up over the delivered tokens prefills only the last one and continues greedily
    follow = e.generate(prompt + got, max_new=8, chunk=8)
    _, last = e.prefix_info()
    assert last == 1
    assert follow == ref[5:13]
    # ill_stop before a request does not leak into it: set_state clears the word
    e.stop()
    e.truncate_cache(0)
    assert e.generate(prompt, max_new=12, chunk=4) == ref[:12]
