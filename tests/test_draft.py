"""CPU tests of the drafting restatement (oracle/draft.py, k_commit_spec drafting,
Shaders.swift:367-412) on known answers, and of the package's n-gram table builder
(instantllm_amd/ngram.py, NGramTable.build) through the oracle's lookup."""
from __future__ import annotations

import numpy as np

from instantllm_amd import ngram
from oracle import draft as D

EOS = (151645, 151643)


def test_self_repetition_continues_a_cycle():
    out = [1, 2, 3, 4, 5, 1, 2, 3, 4]
    assert D.draft(out, [], 4, EOS) == [5, 1, 2]
    # the latest occurrence wins among equally long matches
    out = [9, 7, 8, 6, 1, 7, 8, 6, 2, 7, 8, 6]
    assert D.draft(out, [], 2, EOS) == [2]


def test_self_repetition_needs_three_tokens():
    # a two-token repeat is not enough; nothing else to go on
    assert D.draft([1, 2, 5, 1, 2], [], 4, EOS) == []


def test_prompt_lookup():
    assert D.draft([7, 8], [1, 7, 8, 9, 3], 4, EOS) == [9, 3]


def test_stop_token_ends_drafts_and_nodraft():
    out = [1, 2, 3, EOS[0], 1, 2, 3]
    assert D.draft(out, [], 8, EOS) == [EOS[0]]
    assert D.draft([1, 2, 3, 4, 5, 1, 2, 3, 4], [], 4, EOS, nodraft=True) == []


def test_ngram_table_lookup_round_trip():
    seq = [10, 11, 12, 13, 14]
    table = ngram.build([seq])
    # after the first two tokens, the order-6 context (-1 x 4, 10, 11) knows 12, then 13, 14
    assert D.draft([10, 11], [], 4, EOS, table) == [12, 13, 14]
    assert D.ng_next(table, [-1] * 4 + [10, 11]) == 12
    # an unknown context of every order: no draft from the table
    assert D.ng_next(table, [99, 98, 97, 96, 95, 94]) == -1


def test_ngram_most_frequent_continuation_lowest_id_on_ties():
    table = ngram.build([[5, 6], [5, 7], [5, 7], [8, 9], [8, 3]])
    assert D.ng_next(table, [-1] * 5 + [5]) == 7     # 7 seen twice, 6 once
    assert D.ng_next(table, [-1] * 5 + [8]) == 3     # tie: the lower id
    k = ngram.key([-1] * 5 + [5])
    assert k == D.ng_key([-1] * 5 + [5]) and k & 1


def test_simulate_cycle_accepts_drafts():
    g = [1, 2, 3, 4] * 10
    toks, passes, acc = D.simulate([9, 9], g, 30, 8)
    assert toks == g[:30]
    # every pass commits its accepted drafts and one more token (the last may stop early)
    assert passes + acc >= 30 and acc > 10 and passes < 20


def test_simulate_without_drafts_is_one_token_per_pass():
    rng = np.random.default_rng(0)
    g = [int(t) for t in rng.integers(0, 10**6, 25)]
    toks, passes, acc = D.simulate([3], g, 25, 16)
    assert toks == g and passes == 25 and acc == 0
