"""GPU tests of the learned drafter (ill_ildraft_kernel, k_ildraft Shaders.swift:421-872),
through the C ABI.

* Every pass the drafting kernel sets up equals the oracle's drafts (oracle/ildraft.py, the
  float32 restatement pinned against the reference's Python drafter): the chain of up to
  T - 1 tokens or the best-first tree, given the tokens committed so far.
* Speculative generation with the learned drafter commits exactly the greedy tokens
  (README.md:90-93), and its passes / accepted counts equal the oracle's simulation.

The tables are built from the test model's own greedy outputs (instantllm_amd.ildraft), so
the drafts are often right and both accept and reject paths run.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

from instantllm_amd import synth, illfile as F
from instantllm_amd import ildraft as W
from oracle import ildraft as O

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
from ildraft_corpus import Corpus, mock_encode  # noqa: E402

pytestmark = pytest.mark.gpu

VOCAB = 4096
EMPH = {1: 3.0, 2: 1.5, 17: 2.0, 20: 1.0, 23: 1.5, 36: 0.5, 29: -1.0}


def log(*a):
    print(*a, flush=True)


def _requests(seed, n, vocab):
    rng = np.random.default_rng(seed)
    words = Corpus(seed=1).vocab_words
    out = []
    for _ in range(n):
        pids = [int(t) for t in rng.integers(100, vocab, int(rng.integers(12, 30)))]
        text = " ".join(rng.choice(words, int(rng.integers(4, 9))))
        out.append((pids, text))
    return out


@pytest.fixture(scope="module")
def setup(tmp_path_factory):
    from instantllm_amd.engine import Engine
    d = tmp_path_factory.mktemp("ildraft")
    path = str(d / "q4.ill")
    synth.build_model(path, F.FMT_Q4, seed=2, shape=synth.ModelShape(layers=3, vocab=VOCAB))
    e = Engine(path, max_context=1024, max_pass=16, max_steps=256)
    reqs = _requests(7, 24, VOCAB)
    recs = []
    for pids, text in reqs:
        y = e.generate(pids, max_new=60, chunk=8)
        recs.append({"prompt": text, "pids": pids, "y": y})
    tpath = str(d / "ildraft.bin")
    W.save(tpath, recs, W.TableSpec(pair_min_count=1), W.random_scorer(16, seed=5, emphasis=EMPH), Corpus(seed=1).flags)
    e.load_ildraft(tpath)
    tab = O.Table.load(tpath)
    yield e, tab, reqs
    e.close()


def _oracle_plan(tab, req, vocab, rows, tree):
    d = O.Drafter(tab, req, vocab=vocab)
    if tree:
        return lambda out: ("tree",) + d.tree(out, tree)
    return lambda out: ("chain", d.chain(out, rows - 1))


@pytest.mark.parametrize("tree", [0, 15])
def test_pending_passes_match_oracle(setup, tree):
    """Step by step: after the prompt's commit and after every verify pass, the rows (and the
    tree) the drafting kernel set up equal the oracle's drafts for the committed tokens."""
    e, tab, reqs = setup
    pids, text = reqs[3]
    rows = tree + 1 if tree else 8
    e.set_learned(True, 8, tree)
    e.set_draft_context(pids, text, mock_encode)
    req = O.Req(tab, pids, text, mock_encode)
    dr = O.Drafter(tab, req, vocab=VOCAB)
    e.reset_out_tokens()
    e.set_prompt(pids)
    e.set_state(pos=0, n=len(pids), maxsteps=40, tspec=rows, learned=1)
    e.prefill(pids)
    checked = 0
    for it in range(12):
        st = e.get_state()
        if st["done"]:
            break
        out = [int(t) for t in e.out_tokens()[:st["step"]]]
        mode, nrows, toks, trbuf = e.pending_pass()
        if tree:
            par, tk = dr.tree(out, tree)
            rt, dep, rp = O.tree_rows(par, tk, out[-1])
            log(f"tree pass {it}: rows {nrows} (oracle {len(rt)})")
            assert mode == 2 and toks == rt
            assert list(trbuf[1:1 + nrows]) == dep
            assert list(trbuf[17 + 1:17 + nrows]) == rp[1:]
        else:
            ch = dr.chain(out, rows - 1)
            log(f"chain pass {it}: drafts {toks[1:]} (oracle {ch})")
            assert mode == 1 and toks == [out[-1]] + ch
        checked += 1
        e.spec_pass()
    assert checked >= 4


@pytest.mark.parametrize("tree", [0, 15])
def test_learned_generate_equals_greedy_and_oracle_counts(setup, tree):
    e, tab, reqs = setup
    for k in (0, 5):
        pids, text = reqs[k]
        e.truncate_cache(0)   # compare cold runs
        gx = e.generate(pids, max_new=48 + 16, chunk=8)
        g = gx[:48]
        e.set_learned(True, 8, tree)
        e.set_draft_context(pids, text, mock_encode)
        e.truncate_cache(0)   # compare cold runs
        toks, passes, acc = e.generate_spec(pids, 48, chunk=4)
        assert toks == g
        req = O.Req(tab, pids, text, mock_encode)
        rows = tree + 1 if tree else 8
        _, p_ref, a_ref = O.simulate(pids, gx, 48, _oracle_plan(tab, req, VOCAB, rows, tree))
        log(f"learned {'tree' if tree else 'chain'} req {k}: passes {passes} accepted {acc} (oracle {p_ref} / {a_ref})")
        assert (passes, acc) == (p_ref, a_ref)
        assert acc > 0


def test_learned_unseen_request_and_adaptive(setup):
    """A request the table has never seen (drafts often wrong) with adaptive shapes: the
    output is still exactly greedy."""
    e, tab, _ = setup
    pids, text = _requests(99, 1, VOCAB)[0]
    e.truncate_cache(0)   # compare cold runs
    g = e.generate(pids, max_new=40, chunk=8)
    e.set_learned(True, 8, 15)
    e.set_draft_context(pids, text, mock_encode)
    e.truncate_cache(0)   # compare cold runs
    toks, passes, acc = e.generate_spec(pids, 40, chunk=2, adaptive=True)
    log(f"unseen adaptive: passes {passes} accepted {acc}")
    assert toks == g


def test_context_is_consumed_and_ngram_path_returns(setup):
    """Without a fresh context, generate_spec drafts with the commit's own drafter again."""
    e, tab, reqs = setup
    pids, text = reqs[1]
    e.truncate_cache(0)   # compare cold runs
    g = e.generate(pids, max_new=24, chunk=8)
    e.set_learned(True, 8, 0)
    e.set_draft_context(pids, text, mock_encode)
    e.truncate_cache(0)   # compare cold runs
    t1, _, _ = e.generate_spec(pids, 24, rows=16, chunk=4)
    assert e.get_state()["learned"] == 1
    e.truncate_cache(0)   # compare cold runs
    t2, _, _ = e.generate_spec(pids, 24, rows=16, chunk=4)
    assert e.get_state()["learned"] == 0
    assert t1 == g and t2 == g


def test_learned_fullsize_q4():
    """The full q4 model of seed 2 (vocabulary 151936): learned tree speculation equals greedy."""
    from instantllm_amd.engine import Engine
    import tempfile
    path = synth.cached_model(F.FMT_Q4, 2)
    e = Engine(path, max_context=1024, max_pass=16, max_steps=256)
    try:
        reqs = _requests(11, 6, F.VOCAB)
        recs = []
        for pids, text in reqs:
            recs.append({"prompt": text, "pids": pids, "y": e.generate(pids, max_new=48, chunk=8)})
        with tempfile.TemporaryDirectory() as td:
            tp = str(Path(td) / "t.bin")
            W.save(tp, recs, W.TableSpec(), W.random_scorer(16, seed=5, emphasis=EMPH), {})
            e.load_ildraft(tp)
            tab = O.Table.load(tp)
        pids, text = reqs[2]
        e.truncate_cache(0)   # compare cold runs
        gx = e.generate(pids, max_new=40 + 16, chunk=8)
        e.set_learned(True, 8, 15)
        e.set_draft_context(pids, text, mock_encode)
        e.truncate_cache(0)   # compare cold runs
        toks, passes, acc = e.generate_spec(pids, 40, chunk=4)
        req = O.Req(tab, pids, text, mock_encode)
        _, p_ref, a_ref = O.simulate(pids, gx, 40, _oracle_plan(tab, req, F.VOCAB, 16, 15))
        log(f"full q4 learned tree: passes {passes} accepted {acc} (oracle {p_ref} / {a_ref})")
        assert toks == gx[:40]
        assert (passes, acc) == (p_ref, a_ref)
    finally:
        e.close()


@pytest.fixture(scope="module")
def corpus_engine(tmp_path_factory):
    """An engine (the 3-layer model) with the fixture table of the synthetic request corpus."""
    from instantllm_amd.engine import Engine
    from make_ildraft_fixtures import make_table
    d = tmp_path_factory.mktemp("corpus")
    path = str(d / "q4.ill")
    synth.build_model(path, F.FMT_Q4, seed=2, shape=synth.ModelShape(layers=3, vocab=VOCAB))
    blob, reqs = make_table()
    (d / "corpus.bin").write_bytes(blob)
    e = Engine(path, max_context=1024, max_pass=16, max_steps=256)
    e.load_ildraft(str(d / "corpus.bin"))
    yield e, O.Table(blob), reqs
    e.close()


@pytest.mark.parametrize("tree", [0, 15])
def test_pending_passes_match_oracle_corpus_table(corpus_engine, tree):
    """The fixture table of the synthetic request corpus (300 requests: neighbours, copy
    candidates, associations and space variants all in play; the reference drafter's golden
    vectors pin the oracle on it): each pass's drafts equal the oracle's, request by request."""
    e, tab, reqs = corpus_engine
    rows = tree + 1 if tree else 8
    checked = 0
    for r in reqs[6:10]:
        pids = [t for t in r["pids"] if t < VOCAB]
        e.set_learned(True, 8, tree)
        e.set_draft_context(pids, r["prompt"], mock_encode)
        dr = O.Drafter(tab, O.Req(tab, pids, r["prompt"], mock_encode), vocab=VOCAB)
        e.reset_out_tokens()
        e.set_prompt(pids)
        e.set_state(pos=0, n=len(pids), maxsteps=24, tspec=rows, learned=1)
        e.prefill(pids)
        for _ in range(6):
            st = e.get_state()
            if st["done"]:
                break
            out = [int(t) for t in e.out_tokens()[:st["step"]]]
            mode, nrows, toks, trbuf = e.pending_pass()
            if tree:
                par, tk = dr.tree(out, tree)
                rt, dep, _ = O.tree_rows(par, tk, out[-1])
                assert mode == 2 and toks == rt and list(trbuf[1:1 + nrows]) == dep
            else:
                assert mode == 1 and toks == [out[-1]] + dr.chain(out, rows - 1)
            checked += 1
            e.spec_pass()
    log(f"corpus table, {'tree' if tree else 'chain'}: {checked} passes checked")
    assert checked >= 12
