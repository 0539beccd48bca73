"""CPU tests of the learned drafter's restatement (oracle/ildraft.py) and table writer
(instantllm_amd/ildraft.py) against golden vectors of the reference's own Python drafter
(tools/draft/ildraft.py; written by tests/golden/make_ildraft_fixtures.py).

Tolerances: the reference drafter computes in float64, the engine (and the oracle) in
float32, so probabilities agree to 1e-5 and a draft may differ only where the reference's
two best probabilities at that step are within 1e-5 of each other (a near tie); such steps
are counted and must stay rare.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))
from ildraft_corpus import mock_encode  # noqa: E402
from make_ildraft_fixtures import make_table  # noqa: E402

from oracle import ildraft as O  # noqa: E402

PTOL = 1e-5


@pytest.fixture(scope="module")
def golden():
    g = json.loads((HERE / "golden" / "ildraft_small.json").read_text())
    blob, reqs = make_table()
    assert hashlib.sha256(blob).hexdigest() == g["table_sha256"], "table writer output changed"
    tab = O.Table(blob)
    return tab, reqs, g["requests"]


def test_table_header_and_sections(golden):
    tab, _, _ = golden
    assert (tab.N, tab.M, tab.KNB, tab.MAXM, tab.F, tab.H) == (6, 6, 16, 12, 53, 16)
    for s in ["NGKY", "NGVL", "NGNX", "WDKY", "WDVL", "POST", "DNRM", "SQOF", "SQTK", "CPTK", "CPC1", "CPC2",
              "TFLS", "MLP0", "ASWK", "ASWV", "ASTK"]:
        assert s in tab.sec
    # every section is 8-byte aligned and the n-gram keys ascend
    assert all(off % 8 == 0 for _, off in tab.sec.values())
    keys = sorted(tab.ng)
    assert len(keys) == tab.sec["NGKY"][0]


def test_ctx_key_and_words_known_answers():
    # FNV-1a 64 of b"a" (published test vector) and of the empty string
    assert O.fnv1a64(b"") == 0xCBF29CE484222325
    assert O.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert O.ctx_key([1]) == O.fnv1a64(bytes([1, 1, 0, 0, 0]))
    assert O.prompt_words("Foo bar, FOO baz9 qux-1") == [b"foo", b"bar", b"baz9", b"qux", b"1"]
    assert O.spacevar_words("see src/main.py, v1.2 and x@y!") == ["see", "src/main.py", "v1.2", "and", "x@y"]


def test_request_context_matches_reference(golden):
    tab, reqs, g = golden
    for r, v in zip(reqs, g):
        q = O.Req(tab, r["pids"], r["prompt"], mock_encode)
        assert [list(s) for _, _, s in q.nb] == [s[:80] for s in v["nb_seqs"]]
        np.testing.assert_allclose([float(s) for s, _, _ in q.nb], v["nb_scores"], rtol=1e-6)
        assert q.copy == v["copy"]
        ref_as = {int(k): (x[0], x[1]) for k, x in v["assoc"].items()}
        assert q.as_tok == sorted(ref_as)
        assert [float(x) for x in q.as_max] == [ref_as[t][0] for t in q.as_tok]
        assert q.as_cnt == [ref_as[t][1] for t in q.as_tok]


def _near_tie(top):
    return len(top) >= 2 and abs(top[0][1] - top[1][1]) < PTOL


def test_probs_and_chains_match_reference(golden):
    tab, reqs, g = golden
    ties = mism = steps = 0
    for r, v in zip(reqs, g):
        d = O.Drafter(tab, O.Req(tab, r["pids"], r["prompt"], mock_encode), py_compat=True)
        y = r["y"]
        for i, pv in enumerate(v["pos"], start=1):
            pr = d.probs(y[:i])
            top = pv["top"]
            steps += 1
            assert len(pr) >= len(top)
            for (t, p), (tr, prf) in zip(pr[:3], top):
                assert abs(p - prf) <= PTOL
                if t != tr:
                    assert abs(p - prf) <= PTOL
            ch = d.chain(y[:i], 7)
            if ch != pv["chain"]:
                # the first divergence must be a near tie of the reference at that step
                k = next(j for j in range(min(len(ch), len(pv["chain"]))) if ch[j] != pv["chain"][j])
                ref_top = d.probs(y[:i] + ch[:k])
                assert _near_tie(ref_top), (i, k, ch, pv["chain"])
                ties += 1
            mism += ch != pv["chain"]
    assert steps > 400 and ties <= steps // 50


def test_trees_match_reference(golden):
    tab, reqs, g = golden
    n = 0
    for r, v in zip(reqs, g):
        d = O.Drafter(tab, O.Req(tab, r["pids"], r["prompt"], mock_encode), py_compat=True)
        for tr in v["trees"]:
            par, toks = d.tree(r["y"][:tr["at"]], 15)
            assert (par, toks) == (tr["parents"], tr["tokens"])
            assert all(p < i for i, p in enumerate(par))
            n += 1
    assert n >= 16


def test_features_match_reference(golden):
    """Candidates and the 53 feature rows (ildraft.py `features`) at two positions per
    request; float32 features agree with the reference's float64 ones to 1e-6 (absolute and
    relative: float32 rounding)."""
    tab, reqs, g = golden
    n = 0
    for r, v in zip(reqs, g):
        d = O.Drafter(tab, O.Req(tab, r["pids"], r["prompt"], mock_encode), py_compat=True)
        y = r["y"]
        for i, pv in enumerate(v["pos"], start=1):
            if "feat" not in pv:
                continue
            ob, have, ticks = d._state(y[:i])
            toks, Fm = d.features(ob, have, ticks, y[0])
            assert toks == pv["feat"]["toks"]
            np.testing.assert_allclose(Fm, np.array(pv["feat"]["rows"]), atol=1e-6, rtol=1e-6)
            n += 1
    assert n >= 30


def test_first_unused_threshold_engine_vs_python(golden):
    """The one deliberate difference from the Python drafter: the engine compares the copy
    rate with 0.3f. Engine and Python features differ exactly where a prompt token's rate is
    float32(0.3), and nowhere else."""
    tab, reqs, _ = golden
    seen_diff = False
    for r in reqs:
        q = O.Req(tab, r["pids"], r["prompt"], mock_encode)
        de, dp = O.Drafter(tab, q), O.Drafter(tab, q, py_compat=True)
        y = r["y"]
        for i in range(1, len(y)):
            ob, have, ticks = de._state(y[:i])
            te, fe = de.features(ob, have, ticks, y[0])
            tp, fp = dp.features(ob, have, ticks, y[0])
            assert te == tp
            diff = np.nonzero((fe != fp).any(axis=0))[0]
            assert set(diff.tolist()) <= {37}
            if diff.size:
                seen_diff = True
                assert any(pp == np.float32(0.3) and x not in ob for x, pp in zip(q.P, q.pprop))
    assert float(np.float32(0.3)) > 0.3 and (1 + 0.5) / (3 + 2) == 0.3
    assert seen_diff


def test_scorer_closed_form(golden):
    """The float32 scorer in its fixed order equals the float64 formula
    W2 . relu(W1 x + b1) + b2 + WL . x (ildraft.py:25-26) to float32 rounding."""
    tab, reqs, _ = golden
    d = O.Drafter(tab, O.Req(tab, reqs[0]["pids"], reqs[0]["prompt"], mock_encode))
    y = reqs[0]["y"]
    ob, have, ticks = d._state(y[:5])
    toks, Fm = d.features(ob, have, ticks, y[0])
    sc = d.score(Fm)
    X = Fm.astype(np.float64)
    W1, b1, W2, WL = (a.astype(np.float64) for a in (tab.W1, tab.b1, tab.W2, tab.WL))
    ref = np.maximum(X @ W1.T + b1, 0) @ W2 + float(tab.b2) + X @ WL
    assert len(toks) > 3 and toks == sorted(toks)
    np.testing.assert_allclose(sc, ref, rtol=1e-5, atol=1e-5)


def test_simulate_tree_walk():
    # root's children 5 (node 0) and 6 (node 1); 6's child 7 (node 2)
    plan = ("tree", [-1, -1, 1], [5, 6, 7])
    out, passes, acc = O.simulate([1], [9, 6, 7, 8, 8, 8], 6, lambda o: plan if len(o) == 1 else ("chain", []))
    assert out == [9, 6, 7, 8, 8, 8] and acc == 2 and passes == 4


def test_host_request_context_equals_oracle(golden, tmp_path):
    """The library's request preparation (ill_ildraft_prepare, host code: no GPU) equals the
    oracle's field by field: prompt ids and copy rates, neighbours (float32 scores and their
    80-token sequences), copy candidates and associations."""
    from instantllm_amd.engine import DraftTable
    tab, reqs, _ = golden
    p = tmp_path / "t.bin"
    blob, _ = make_table()
    p.write_bytes(blob)
    d = DraftTable(str(p))
    try:
        for r in reqs:
            q = d.prepare(r["pids"], r["prompt"], mock_encode)
            o = O.Req(tab, r["pids"], r["prompt"], mock_encode)
            assert q["np"] == len(o.P) and q["P"][:q["np"]].tolist() == o.P
            assert q["pprop"][:q["np"]].tolist() == [float(x) for x in o.pprop]
            assert q["nnb"] == len(o.nb)
            for k, (sc, _, seq) in enumerate(o.nb):
                assert q["nbScore"][k] == sc
                assert q["nbTok"][q["nbOff"][k]:q["nbOff"][k + 1]].tolist() == seq
            n = q["ncopy"]
            assert q["copyTok"][:n].tolist() == o.copy
            assert q["copyInP"][:n].tolist() == [int(x) for x in o.copy_inp]
            assert q["copyPt"][:n].tolist() == [float(x) for x in o.copy_pt]
            f33 = [float(O._logf(pt / O.F32(O.F32(1) - pt)) / O.F32(4)) for pt in o.copy_pt]
            assert q["copyF33"][:n].tolist() == f33
            assert q["asTok"][:q["nas"]].tolist() == o.as_tok
            assert q["asMax"][:q["nas"]].tolist() == [float(x) for x in o.as_max]
            assert q["asCnt"][:q["nas"]].tolist() == o.as_cnt
        # no tokenizer: no space-variant candidates, only the prompt ids
        q = d.prepare(reqs[0]["pids"], reqs[0]["prompt"], None)
        assert q["copyTok"][:q["ncopy"]].tolist() == sorted(set(reqs[0]["pids"]))
    finally:
        d.close()


def test_table_errors(tmp_path):
    from instantllm_amd.engine import DraftTable, IllError
    blob, _ = make_table()
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"NOTADRAFT" + blob[9:])
    with pytest.raises(IllError, match="not an ILDRAFT1 table"):
        DraftTable(str(bad))
    trunc = tmp_path / "trunc.bin"
    trunc.write_bytes(blob[: len(blob) // 2])
    with pytest.raises(IllError, match="out of range"):
        DraftTable(str(trunc))
    cfg = bytearray(blob)
    cfg[32:36] = (54).to_bytes(4, "little")   # F = 54 features
    c = tmp_path / "cfg.bin"
    c.write_bytes(bytes(cfg))
    with pytest.raises(IllError, match="unsupported drafter config"):
        DraftTable(str(c))
    with pytest.raises(IllError, match="cannot read"):
        DraftTable(str(tmp_path / "missing.bin"))


# ---- the reference's own shipped table (tools/draft/ildraft-q4.bin) ----------------------
REAL = Path("/root/reference/tools/draft/ildraft-q4.bin")


@pytest.fixture(scope="module")
def real():
    if not REAL.exists():
        pytest.skip("the reference tree (its shipped drafter table) is not present")
    g = json.loads((HERE / "golden" / "ildraft_real.json").read_text())
    blob = REAL.read_bytes()
    assert hashlib.sha256(blob).hexdigest() == g["table_sha256"]
    return O.Table(blob), g["requests"]


def test_real_table_context_features_and_drafts(real):
    """On the reference's trained table: request context, feature rows, probabilities,
    chains and trees of the restatement equal the reference drafter's (Python-drafter mode:
    no engine caps, the 0.3 comparison in float64)."""
    tab, g = real
    ties = steps = nfeat = 0
    for v in g:
        q = O.Req(tab, v["pids"], v["prompt"], mock_encode, python=True)
        assert [list(s) for _, _, s in q.nb] == v["nb_seqs"]
        np.testing.assert_allclose([float(s) for s, _, _ in q.nb], v["nb_scores"], rtol=1e-6)
        assert q.copy == v["copy"]
        ref_as = {int(k): (x[0], x[1]) for k, x in v["assoc"].items()}
        assert q.as_tok == sorted(ref_as) and q.as_cnt == [ref_as[t][1] for t in q.as_tok]
        d = O.Drafter(tab, q, py_compat=True)
        y = v["y"]
        for i, pv in enumerate(v["pos"], start=1):
            steps += 1
            pr = d.probs(y[:i])
            for (t, p), (tr, prf) in zip(pr[:3], pv["top"]):
                assert abs(p - prf) <= PTOL
            if "feat" in pv:
                ob, have, ticks = d._state(y[:i])
                toks, Fm = d.features(ob, have, ticks, y[0])
                assert toks == pv["feat"]["toks"]
                np.testing.assert_allclose(Fm, np.array(pv["feat"]["rows"]), atol=1e-6, rtol=1e-6)
                nfeat += 1
            ch = d.chain(y[:i], 7)
            if ch != pv["chain"]:
                k = next(j for j in range(min(len(ch), len(pv["chain"]))) if ch[j] != pv["chain"][j])
                assert _near_tie(d.probs(y[:i] + ch[:k])), (i, k, ch, pv["chain"])
                ties += 1
        for tr in v["trees"]:
            assert d.tree(y[:tr["at"]], 15) == (tr["parents"], tr["tokens"])
    assert steps > 100 and nfeat >= 20 and ties <= steps // 50


def test_real_table_host_context_equals_oracle(real):
    """The library loads the reference's table (its checks pass) and prepares the engine's
    request context as the oracle does (80-token neighbour sequences)."""
    from instantllm_amd.engine import DraftTable
    tab, g = real
    d = DraftTable(str(REAL))
    try:
        for v in g:
            q = d.prepare(v["pids"], v["prompt"], mock_encode)
            o = O.Req(tab, v["pids"], v["prompt"], mock_encode)
            assert q["nnb"] == len(o.nb)
            for k, (sc, _, seq) in enumerate(o.nb):
                assert q["nbScore"][k] == sc
                assert q["nbTok"][q["nbOff"][k]:q["nbOff"][k + 1]].tolist() == seq
            assert q["copyTok"][:q["ncopy"]].tolist() == o.copy
            assert q["copyPt"][:q["ncopy"]].tolist() == [float(x) for x in o.copy_pt]
            assert q["asTok"][:q["nas"]].tolist() == o.as_tok
            assert q["asMax"][:q["nas"]].tolist() == [float(x) for x in o.as_max]
    finally:
        d.close()
