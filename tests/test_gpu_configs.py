"""GPU parity of the BASELINE configurations at their own sizes, through the C ABI.

* config 0: the full-size f16 model of seed 0, a 48-token prompt and 32 greedy tokens:
  every step's logits within relative L2 1e-2 of the fp32 oracle fed the engine's own
  tokens, and teacher-forced greedy agreement >= 99% at vocabulary 151936;
* config 1: the four stand-alone q4 GEMV shapes (QKV, gate/up, down, and the lm_head
  151936 x 896 with its argmax epilogue on the one-slice kernel) against the float64
  dequantization;
* config 4's long context (q8, f16 and q4): a 4032-token prefill, then decode steps up
  to 4096 attended positions against the oracle, and a 16-row tree pass near 4096 whose rows equal the
  1-row steps along their paths bit for bit (the attention split over four workgroups per
  (row, head) and their combine);
* the decode-step invariant: the logits of N 1-row decode steps (single launches and a
  captured graph) equal, bit for bit, the rows of one chain pass over the same tokens.
"""
from __future__ import annotations

import numpy as np
import pytest

from instantllm_amd import synth, illfile as F
from oracle import illread, qwen, metrics, tree as T

pytestmark = pytest.mark.gpu

REL_L2_TOL = 1e-2
NO_EOS = (-5, -5)


def log(*a):
    print(*a, flush=True)


# ---- config 0 ---------------------------------------------------------------------------

def test_config0_fullsize_f16_greedy_32():
    from instantllm_amd.engine import Engine
    log("config 0: full f16 model, seed 0 (generate or reuse)")
    path = synth.cached_model(F.FMT_F16, 0)
    log("config 0: oracle load (dequantized fp32)")
    m = qwen.Model(illread.load(path))
    prompt = [int(t) for t in np.random.default_rng(0).integers(0, F.VOCAB, size=48)]
    e = Engine(path, max_context=256, max_pass=16, max_steps=64)
    try:
        e.reset_out_tokens()
        e.set_state(pos=0, n=len(prompt), maxsteps=32, eos=NO_EOS)
        log("config 0: prefill 48 + 31 decode steps, logits of every step")
        e.prefill(prompt, write_logits=True)
        cache = m.new_cache(96)
        errs = [metrics.rel_l2(e.read_logits(0), m.forward(prompt, cache))]
        toks = [int(e.out_tokens()[0])]
        for s in range(31):
            e.decode_step(write_logits=True)
            lg = e.read_logits(0)
            errs.append(metrics.rel_l2(lg, m.forward([toks[-1]], cache)))
            nxt = int(e.out_tokens()[s + 1])
            assert nxt == int(np.argmax(lg)), s
            toks.append(nxt)
        log(f"config 0: rel L2 max {max(errs):.2e} median {np.median(errs):.2e}")
        assert max(errs) <= REL_L2_TOL, errs
        am, _ = m.teacher_forced(prompt, toks)
        agree, n = metrics.forced_agreement(toks, am)
        log(f"config 0: teacher-forced agreement {agree}/{n}")
        assert agree / n >= 0.99, (agree, n)
    finally:
        e.close()


# ---- config 1 ---------------------------------------------------------------------------

def _gemv_ref(codes, sb, x, gamma):
    xx = x.astype(np.float64)
    if gamma is not None:
        xx = qwen.rmsnorm(xx[None, :], gamma.astype(np.float64))[0]
    rows = codes.shape[0]
    y = np.empty(rows, np.float64)
    for r0 in range(0, rows, 16384):   # dequantize in row blocks (the lm_head is 136 M weights)
        w = illread.dequant_q4(codes[r0:r0 + 16384], sb[r0:r0 + 16384]).astype(np.float64)
        y[r0:r0 + 16384] = w @ xx
    return y


@pytest.mark.parametrize("name,rows,K,norm,amax,kernel_slices", [
    ("qkv", 1152, 896, True, False, None),
    ("gate_up", 9728, 896, True, False, None),
    ("down", 896, 4864, False, False, None),
    ("lm_head", 151936, 896, True, True, 1),   # one-slice kernel + argmax epilogue
])
def test_config1_gemv_shapes(name, rows, K, norm, amax, kernel_slices):
    from instantllm_amd.engine import Gemv
    codes, sb = synth.microbench_q4(1, rows, K)
    x, gamma = synth.microbench_x(1, K)
    x = x[0]
    log(f"config 1 {name}: {rows} x {K}")
    g = Gemv(codes, np.ascontiguousarray(sb).view(np.uint32).reshape(rows, K // 64), copies=2)
    try:
        info = g.info()
        if kernel_slices is not None:
            assert info["slices"] == kernel_slices, info
        y, am, _ = g.run(x, gamma if norm else None, iters=3, argmax=amax)
    finally:
        g.close()
    ref = _gemv_ref(codes, sb, x, gamma if norm else None)
    err = metrics.rel_l2(y, ref)
    log(f"config 1 {name}: rel L2 {err:.2e}, slices {info['slices']}")
    assert err <= REL_L2_TOL
    if amax:
        assert am == int(np.argmax(y))   # lowest index of the kernel's own maximum
        assert ref[am] >= ref.max() - 1e-3 * np.abs(ref).max()


# ---- config 4 at 4096 positions ----------------------------------------------------------

@pytest.mark.parametrize("fmt", [F.FMT_Q8, F.FMT_F16, F.FMT_Q4], ids=["q8", "f16", "q4"])
def test_config4_context_4096(tmp_path, fmt):
    """4032-token prefill, decode steps up to 4096 attended positions with the oracle's
    logits at every step, then a 16-row tree pass at 4064 whose rows equal 1-row steps
    along their paths bit for bit."""
    from instantllm_amd.engine import Engine
    vocab = 4096
    path = str(tmp_path / "m.ill")
    synth.build_model(path, fmt, seed=4, shape=synth.ModelShape(layers=3, vocab=vocab))
    m = qwen.Model(illread.load(path))
    e = Engine(path, max_context=4160, max_pass=16, max_steps=256)
    try:
        rng = np.random.default_rng(4)
        ctx = [int(t) for t in rng.integers(0, vocab, size=4032)]
        e.reset_out_tokens()
        e.set_state(pos=0, n=len(ctx), maxsteps=200, eos=NO_EOS)
        log(f"format {fmt}: prefill 4032")
        e.prefill(ctx, write_logits=True)
        cache = m.new_cache(4160)
        for c0 in range(0, 4032, 1008):   # oracle prefill in chunks (attention memory)
            ref = m.forward(ctx[c0:c0 + 1008], cache)
        assert metrics.rel_l2(e.read_logits(0), ref) <= REL_L2_TOL
        tok = int(e.out_tokens()[0])
        log(f"format {fmt}: 64 decode steps, positions 4032 .. 4095")
        for s in range(64):
            e.decode_step(write_logits=True)
            lg = e.read_logits(0)
            err = metrics.rel_l2(lg, m.forward([tok], cache))
            assert err <= REL_L2_TOL, (s, err)
            tok = int(e.out_tokens()[s + 1])
            assert tok == int(np.argmax(lg))
        assert e.get_state()["pos"] == 4096
        # the cache below 4064 is the decode's context: a tree pass there
        pos0 = 4064
        tr = synth.random_tree(rng, 16, vocab)
        e.set_state(pos=pos0, n=16, maxsteps=200, eos=NO_EOS)
        log(f"format {fmt}: tree pass at {pos0}")
        e.verify_pass(16, tree=tr, write_logits=True)
        rows = np.stack([e.read_logits(r) for r in range(16)])
        toks = tr[T.TR_TOK:T.TR_TOK + 16]
        for p in T.paths(tr)[:4]:
            for k, r in enumerate(p):
                e.set_state(pos=pos0 + k, n=1, maxsteps=200, eos=NO_EOS)
                e.prefill([int(toks[r])], write_logits=True)
                one = e.read_logits(0)
                assert np.array_equal(one.view(np.uint32), rows[r].view(np.uint32)), (p, k, r)
    finally:
        e.close()


# ---- the decode step against a chain pass --------------------------------------------------

def _decode_vs_chain(e, prompt, nsteps=15):
    """Logits of `nsteps` decode steps (single launches), of the same steps replayed from a
    captured graph (the last one), and of one chain pass over [t0, g1 .. g_nsteps-1]."""
    e.reset_out_tokens()
    e.set_state(pos=0, n=len(prompt), maxsteps=64, eos=NO_EOS)
    e.prefill(prompt)
    pos0 = e.get_state()["pos"]
    t0 = int(e.out_tokens()[0])
    steps = []
    for s in range(nsteps):
        e.decode_step(write_logits=True)
        steps.append(e.read_logits(0))
    g = [int(t) for t in e.out_tokens()[1:nsteps + 1]]
    # the same steps again: the first as a 1-row pass on t0 (it sets the next input), the
    # others replayed from a captured graph; the graph's last step's logits
    e.reset_out_tokens()
    e.set_state(pos=pos0, n=1, maxsteps=64, eos=NO_EOS)
    e.prefill([t0], write_logits=True)
    assert np.array_equal(e.read_logits(0).view(np.uint32), steps[0].view(np.uint32))
    e.capture_steps(nsteps - 1)
    e.launch_graph(write_logits=True)
    e.sync()
    graph_last = e.read_logits(0)
    assert [int(t) for t in e.out_tokens()[:nsteps]] == g
    # one chain pass over the same rows
    chain = [t0] + g[: nsteps - 1]
    e.set_state(pos=pos0, n=nsteps, maxsteps=64, eos=NO_EOS)
    e.verify_pass(nsteps, toks=chain, write_logits=True)
    rows = [e.read_logits(r) for r in range(nsteps)]
    return steps, graph_last, rows


@pytest.mark.parametrize("nsteps", [15, 4, 3, 2])
def test_decode_steps_equal_chain_pass_rows_small(nsteps):
    """Small q4 model, prompt of 58 (the steps cross the 64-position chunk boundary); chains
    of 15, 4 and 3 rows (the 16-row kernel) and of 2 rows (the 4-row kernel)."""
    from instantllm_amd.engine import Engine
    import tempfile
    import os
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.ill")
        synth.build_model(path, F.FMT_Q4, seed=2, shape=synth.ModelShape(layers=3, vocab=4096))
        e = Engine(path, max_context=1024, max_pass=16, max_steps=256)
        try:
            prompt = [int(t) for t in np.random.default_rng(21).integers(0, 4096, size=58)]
            steps, graph_last, rows = _decode_vs_chain(e, prompt, nsteps)
        finally:
            e.close()
    for r in range(len(rows)):
        assert np.array_equal(steps[r].view(np.uint32), rows[r].view(np.uint32)), r
    assert np.array_equal(graph_last.view(np.uint32), steps[-1].view(np.uint32))


def test_decode_steps_equal_chain_pass_rows_fullsize():
    """The benchmarked path: full q4 model of seed 2, prefix 256 (config 2)."""
    from instantllm_amd.engine import Engine
    path = synth.cached_model(F.FMT_Q4, 2)
    e = Engine(path, max_context=1024, max_pass=16, max_steps=256)
    try:
        prompt = [int(t) for t in np.random.default_rng(2).integers(0, F.VOCAB, size=256)]
        log("full q4: 15 decode steps, graph replay, chain pass at 256")
        steps, graph_last, rows = _decode_vs_chain(e, prompt)
    finally:
        e.close()
    for r in range(len(rows)):
        assert np.array_equal(steps[r].view(np.uint32), rows[r].view(np.uint32)), r
    assert np.array_equal(graph_last.view(np.uint32), steps[-1].view(np.uint32))
