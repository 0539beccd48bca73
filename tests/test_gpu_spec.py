"""GPU tests of speculative decoding with on-device drafting, through the C ABI.

The invariant of the reference (README.md:90-93): speculation never changes the output, so a
speculative request commits exactly the plain greedy tokens. Both runs start from a cold
prefix cache (ill_truncate_cache): a reused prefix moves where the prompt's last tokens are
computed, which may resolve a near tie differently. The device's drafting
(k_commit_spec, Shaders.swift:367-412) is checked end to end against the oracle's
restatement: given the greedy continuation, oracle.draft.simulate predicts every pass's
drafts and accepted prefix, so the State's passes / accepted counters must equal it.
"""
from __future__ import annotations

import numpy as np
import pytest

from instantllm_amd import synth, illfile as F, ngram
from oracle import draft as D

pytestmark = pytest.mark.gpu

VOCAB = 4096


def log(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def q4_engine(tmp_path_factory):
    from instantllm_amd.engine import Engine
    path = str(tmp_path_factory.mktemp("spec") / "q4.ill")
    synth.build_model(path, F.FMT_Q4, seed=2, shape=synth.ModelShape(layers=3, vocab=VOCAB))
    e = Engine(path, max_context=1024, max_pass=16, max_steps=256)
    yield e
    e.close()


def _prompt(seed, n=20):
    return [int(t) for t in np.random.default_rng(seed).integers(0, VOCAB, size=n)]


@pytest.mark.parametrize("rows", [16, 4])
def test_spec_generate_equals_greedy_and_oracle_counts(q4_engine, rows):
    e = q4_engine
    e.load_ngram(None)
    prompt = _prompt(100 + rows)
    e.truncate_cache(0)   # compare cold runs
    gx = e.generate(prompt, max_new=48 + 16, chunk=8)   # 16 more for the last pass's drafts
    g = gx[:48]
    log(f"rows {rows}: greedy {g[:12]}...")
    e.truncate_cache(0)   # compare cold runs
    toks, passes, acc = e.generate_spec(prompt, 48, rows=rows, chunk=4)
    assert toks == g
    _, p_ref, a_ref = D.simulate(prompt, gx, 48, rows)
    log(f"rows {rows}: passes {passes} accepted {acc} (oracle {p_ref} / {a_ref})")
    assert (passes, acc) == (p_ref, a_ref)


def test_spec_with_ngram_table_accepts_drafts(q4_engine):
    e = q4_engine
    prompt = _prompt(7)
    e.truncate_cache(0)   # compare cold runs
    gx = e.generate(prompt, max_new=64 + 16, chunk=8)
    g = gx[:64]
    table = ngram.build([g])
    e.load_ngram(table)
    try:
        e.truncate_cache(0)   # compare cold runs
        toks, passes, acc = e.generate_spec(prompt, 64, rows=16, chunk=4)
    finally:
        e.load_ngram(None)
    assert toks == g
    _, p_ref, a_ref = D.simulate(prompt, gx, 64, 16, table=table)
    log(f"n-gram table: passes {passes} accepted {acc} (oracle {p_ref} / {a_ref})")
    assert (passes, acc) == (p_ref, a_ref)
    assert acc > 0 and passes < 64


def test_graph_chained_passes_equal_single_passes(q4_engine):
    """Passes replayed from one hipGraph (each taking its rows from the commit before it)
    equal the same passes launched one by one."""
    e = q4_engine
    prompt = _prompt(8)
    e.truncate_cache(0)   # compare cold runs
    g = e.generate(prompt, max_new=40, chunk=8)
    table = ngram.build([g[:20]])   # drafts right for the first half, then on their own
    e.load_ngram(table)
    try:
        e.truncate_cache(0)   # compare cold runs
        toks_g, p_g, a_g = e.generate_spec(prompt, 40, rows=16, chunk=3)
        e.reset_out_tokens()
        e.set_prompt(prompt)
        e.set_state(pos=0, n=len(prompt), maxsteps=40, tspec=16)
        e.prefill(prompt)
        for _ in range(40):
            if e.get_state()["done"]:
                break
            e.spec_pass()
        st = e.get_state()
    finally:
        e.load_ngram(None)
    toks_s = [int(t) for t in e.out_tokens()[:40]]
    assert toks_g == g and toks_s == g
    assert (st["passes"], st["accepted"]) == (p_g, a_g)


def test_nodraft_passes_are_one_row(q4_engine):
    e = q4_engine
    prompt = _prompt(9)
    e.truncate_cache(0)   # compare cold runs
    g = e.generate(prompt, max_new=12, chunk=4)
    e.reset_out_tokens()
    e.set_prompt(prompt)
    e.set_state(pos=0, n=len(prompt), maxsteps=12, tspec=16, nodraft=1)
    e.prefill(prompt)
    for _ in range(12):
        if e.get_state()["done"]:
            break
        e.spec_pass()
    st = e.get_state()
    assert [int(t) for t in e.out_tokens()[:12]] == g
    assert st["passes"] == 12 and st["accepted"] == 0


def test_adaptive_shapes_keep_the_output(q4_engine):
    e = q4_engine
    prompt = _prompt(10)
    e.truncate_cache(0)   # compare cold runs
    g = e.generate(prompt, max_new=48, chunk=8)
    e.truncate_cache(0)   # compare cold runs
    toks, _, _ = e.generate_spec(prompt, 48, rows=16, chunk=2, adaptive=True)
    assert toks == g


@pytest.mark.parametrize("fmt", [F.FMT_Q8, F.FMT_F16], ids=["q8g32", "f16"])
def test_spec_layer_by_layer_formats_chain_on_the_device(tmp_path, fmt):
    """q8 and f16 speculative passes chained in hipGraphs (Engine.swift:991-1013 encodes
    every format's passes ahead): the tokens are greedy's and the pass and accept counts the
    oracle's simulation; the same passes launched one by one give the same tokens and counts;
    a captured graph of passes equals them too (adaptive shapes included)."""
    from instantllm_amd.engine import Engine
    path = str(tmp_path / "m.ill")
    synth.build_model(path, fmt, seed=4, shape=synth.ModelShape(layers=3, vocab=VOCAB), q8_group=32)
    e = Engine(path, max_context=1024, max_pass=16, max_steps=128)
    try:
        prompt = _prompt(11)
        e.truncate_cache(0)   # compare cold runs
        gx = e.generate(prompt, max_new=32 + 16, chunk=8)
        g = gx[:32]
        table = ngram.build([g[:20]])   # drafts right for the first part, then on their own
        e.load_ngram(table)
        e.truncate_cache(0)   # compare cold runs
        toks, passes, acc = e.generate_spec(prompt, 32, rows=8, chunk=4)
        assert toks == g
        assert (passes, acc) == D.simulate(prompt, gx, 32, 8, table=table)[1:]
        e.truncate_cache(0)
        toks_a, _, _ = e.generate_spec(prompt, 32, rows=16, chunk=3, adaptive=True)
        assert toks_a == g
        # single passes, then one captured graph of the same passes
        for graph in (False, True):
            e.truncate_cache(0)
            e.reset_out_tokens()
            e.set_prompt(prompt)
            e.set_state(pos=0, n=len(prompt), maxsteps=32, tspec=8)
            e.prefill(prompt)
            if graph:
                e.capture_spec(passes)
                e.launch_graph()
                e.sync()
            else:
                for _ in range(passes):
                    if e.get_state()["done"]:
                        break
                    e.spec_pass()
            st = e.get_state()
            assert [int(t) for t in e.out_tokens()[:32]] == g, graph
            assert (st["passes"], st["accepted"]) == (passes, acc), graph
    finally:
        e.load_ngram(None)
        e.close()


def test_spec_fullsize_q4():
    """The full model of seed 2: speculative tokens equal greedy ones."""
    from instantllm_amd.engine import Engine
    path = synth.cached_model(F.FMT_Q4, 2)
    e = Engine(path, max_context=1024, max_pass=16, max_steps=256)
    try:
        prompt = [int(t) for t in np.random.default_rng(2).integers(0, F.VOCAB, size=64)]
        e.truncate_cache(0)   # compare cold runs
        gx = e.generate(prompt, max_new=48 + 16, chunk=8)
        g = gx[:48]
        table = ngram.build([g])
        e.load_ngram(table)
        e.truncate_cache(0)   # compare cold runs
        toks, passes, acc = e.generate_spec(prompt, 48, rows=16, chunk=4)
    finally:
        e.close()
    log(f"full q4: passes {passes} accepted {acc}")
    assert toks == g
    assert (passes, acc) == D.simulate(prompt, gx, 48, 16, table=table)[1:]


# ---- prefix reuse across requests (Engine.swift:788-838, :929-933) ------------------------

def test_prefix_reuse_prefills_only_the_new_tokens(q4_engine):
    e = q4_engine
    prompt = _prompt(12, 30)
    first = e.generate(prompt, max_new=10, chunk=4)
    cached, pre = e.prefix_info()
    assert pre == 30 and cached == 30 + 10 - 1
    # a follow-up prompt extending the conversation reuses the cached K/V
    prompt2 = prompt + first[:9] + _prompt(13, 5)
    out2 = e.generate(prompt2, max_new=12, chunk=4)
    assert e.prefix_info()[1] == 5
    # the same answer as from a cold cache for this request (a pass outside generate forgets
    # the prefix; a reused prefix may resolve a near tie differently in general)
    e.reset_out_tokens()
    e.set_state(pos=0, n=4, maxsteps=4)
    e.prefill(prompt[:4])
    assert e.prefix_info()[0] == 0
    cold = e.generate(prompt2, max_new=12, chunk=4)
    assert e.prefix_info()[1] == len(prompt2)
    assert out2 == cold
    # the same prompt again: only its last token is prefilled; speculative calls reuse too
    again, _, _ = e.generate_spec(prompt2, 12, rows=8, chunk=4)
    assert e.prefix_info()[1] == 1 and again == cold


def test_prefix_save_and_load(q4_engine, tmp_path):
    e = q4_engine
    prompt = _prompt(14, 40)
    ref = e.generate(prompt, max_new=16, chunk=4)
    f = str(tmp_path / "prefix.bin")
    e.save_prefix(f, prompt)
    # clobber the cache, then load the saved prefix: generation continues from it
    e.reset_out_tokens()
    e.set_state(pos=0, n=8, maxsteps=4)
    e.prefill(_prompt(15, 8))
    toks = e.load_prefix(f)
    assert toks == prompt and e.prefix_info()[0] == 40
    out = e.generate(prompt, max_new=16, chunk=4)
    assert e.prefix_info()[1] == 1 and out == ref


def test_adaptive_levels_keep_the_output(q4_engine):
    """Requests whose drafts mostly miss walk the adaptive levels (16 rows, 4-row chains,
    one-row passes with 4-row probes; graphs per kernel instantiation): the tokens stay
    greedy."""
    e = q4_engine
    e.load_ngram(None)
    for seed in (31, 32):
        prompt = _prompt(seed)
        e.truncate_cache(0)   # compare cold runs
        g = e.generate(prompt, max_new=96, chunk=8)
        e.truncate_cache(0)   # compare cold runs
        toks, passes, acc = e.generate_spec(prompt, 96, rows=16, chunk=2, adaptive=True)
        log(f"adaptive seed {seed}: passes {passes} accepted {acc}")
        assert toks == g


def test_pass_wider_than_the_kernel_is_refused(q4_engine):
    """A pending pass with more rows than the instantiation a graph was captured for is
    refused on the device (every workgroup leaves after reading the header) and reported;
    the engine keeps working."""
    from instantllm_amd.engine import IllError
    e = q4_engine
    prompt = _prompt(41)
    e.truncate_cache(0)   # compare cold runs
    gx = e.generate(prompt, max_new=40, chunk=8)
    e.load_ngram(ngram.build([gx]))
    try:
        e.reset_out_tokens()
        e.set_prompt(prompt)
        e.set_state(pos=0, n=len(prompt), maxsteps=32, tspec=16)
        e.prefill(prompt)                      # the commit drafts up to 15 tokens (table)
        mode, nrows, _, _ = e.pending_pass()
        assert nrows > 4
        st = e.get_state()
        st["tspec"] = 2
        e.set_state(**st)
        e.capture_spec(1)                      # a graph of the 4-row kernel (2-row passes)
        e.launch_graph()
        with pytest.raises(IllError, match="more rows than its kernel"):
            e.sync()                           # reports the device's error
    finally:
        e.load_ngram(None)
    assert e.generate(prompt, max_new=24, chunk=8) == gx[:24]


def test_out_of_vocabulary_draft_sources_are_refused(q4_engine, tmp_path):
    """The drafter embeds what the n-gram table and the prompt propose in the next pass, so
    tokens outside the model's vocabulary are refused when the table or prompt is handed
    over; a drafter table that fails to load leaves the engine with no learned drafter (it
    then drafts with the commit's own drafter and keeps working)."""
    from instantllm_amd.engine import IllError
    e = q4_engine
    prompt = _prompt(43)
    e.truncate_cache(0)
    gx = e.generate(prompt, max_new=24, chunk=8)
    t = ngram.build([gx])
    slot = int(np.flatnonzero(t["key"] != 0)[0])
    t["next"][slot] = VOCAB            # one past the last token
    with pytest.raises(IllError, match="outside the vocabulary"):
        e.load_ngram(t)
    t["next"][slot] = -3
    with pytest.raises(IllError, match="outside the vocabulary"):
        e.load_ngram(t)
    with pytest.raises(IllError, match="out of range"):
        e.set_prompt(prompt[:5] + [VOCAB + 7] + prompt[5:])
    bad = tmp_path / "bad.ildraft"
    bad.write_bytes(b"not a table")
    with pytest.raises(IllError):
        e.load_ildraft(str(bad))
    e.load_ngram(None)
    e.truncate_cache(0)
    toks, _, _ = e.generate_spec(prompt, 16, rows=4, chunk=4)
    assert toks == gx[:16]
