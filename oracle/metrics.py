"""Comparison measures of the oracle harness.

* `topk`: top-k [[id, logit]] sorted by logit descending, ties by lower id
  (`tools/reference/refcommon.py:85-94`).
* `argmax_lowest`: greedy pick, exact ties to the lowest id (`qwen_ref.py:206`).
* `rel_l2`: per-step relative L2 error, the north-star gate (<= 1e-2).
* `compare_logits`: max/mean |d|, top-1 and top-5 overlap (`compare.py:59-71`).
* `forced_agreement`: teacher-forced agreement of per-step argmaxes (`compare.py:99-109`).
"""
from __future__ import annotations

import numpy as np


def topk(logits: np.ndarray, k: int) -> list[list]:
    logits = np.asarray(logits)
    idx = np.argpartition(-logits, k)[:k]
    kth = logits[idx].min()
    idx = np.nonzero(logits >= kth)[0]
    order = np.lexsort((idx, -logits[idx].astype(np.float64)))
    idx = idx[order][:k]
    return [[int(i), float(logits[i])] for i in idx]


def argmax_lowest(logits: np.ndarray) -> int:
    return int(np.argmax(np.asarray(logits)))


def rel_l2(a: np.ndarray, ref: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(a - ref) / max(np.linalg.norm(ref), 1e-30))


def compare_logits(eng: np.ndarray, gold: np.ndarray) -> dict:
    e = np.asarray(eng, np.float64)
    g = np.asarray(gold, np.float64)
    d = np.abs(e - g)
    g5 = [t for t, _ in topk(g, 5)]
    e5 = [t for t, _ in topk(e, 5)]
    return dict(max_abs=float(d.max()), mean_abs=float(d.mean()), rel_l2=rel_l2(e, g),
                top1=g5[0] == e5[0], top5_overlap=len(set(g5) & set(e5)),
                nonfinite=int((~np.isfinite(e)).sum()))


def forced_agreement(golden_seq: list[int], forced_argmax: list[int]) -> tuple[int, int]:
    """(agree, steps) over the golden sequence; missing engine steps count as misses."""
    fa = list(forced_argmax)[: len(golden_seq)]
    agree = sum(1 for a, b in zip(golden_seq, fa) if a == b)
    return agree, len(golden_seq)


def margin(logits: np.ndarray) -> float:
    t = topk(logits, 2)
    return t[0][1] - t[1][1]
