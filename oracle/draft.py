"""CPU restatement of speculative decoding with drafting (test infrastructure only).

* `draft`: the drafting of k_commit_spec (Sources/Engine/Shaders.swift:367-412), written as
  the reference's single-thread loops: up to T - 1 drafts, each from the first source with a
  guess -- self-repetition (the latest earlier occurrence of the longest output suffix of
  3..8 tokens, continued; :386-391), the n-gram table (`ng_next`, :72-86), prompt lookup
  (the token after the latest longest 1..4-token match of the output suffix in the last
  <= 256 prompt tokens; :393-399); each draft is appended to the output, a stop token ends
  the drafts (:400-406).
* `simulate`: a whole speculative request given the model's greedy continuation: the
  prompt's commit (pass 1, no drafts accepted), then chain passes over [last, drafts...]
  accepting the longest prefix of drafts that equals the greedy tokens (:305-333), with the
  passes / accepted counters of the State (:297, :319).

The n-gram lookup reads a table in the NGramTable layout (`instantllm_amd.ngram.ENTRY`).
"""
from __future__ import annotations

NG_SLOTS = 1 << 20
NG_MAXN = 6
OB_MAX = 256
M64 = (1 << 64) - 1


def ng_key(ctx) -> int:
    """Shaders.swift:66-70."""
    h = 0xCBF29CE484222325 ^ len(ctx)
    for t in ctx:
        h = h ^ (((t & 0xFFFFFFFF) + 0x9E3779B97F4A7C15) & M64)
        h = (h * 0x100000001B3) & M64
        h = h ^ (h >> 29)
    return h | 1


def ng_next(table, hist) -> int:
    """Most frequent continuation of the longest known context of `hist` (orders 6..1)."""
    if table is None:
        return -1
    keys, nexts = table["key"], table["next"]
    for n in range(min(NG_MAXN, len(hist)), 0, -1):
        k = ng_key(hist[len(hist) - n:])
        slot = (k >> 12) & (NG_SLOTS - 1)
        for _ in range(16):
            ek = int(keys[slot])
            if ek == 0:
                break
            if ek == k:
                return int(nexts[slot])
            slot = (slot + 1) & (NG_SLOTS - 1)
    return -1


def draft(out, prompt, T, eos, table=None, nodraft=False) -> list[int]:
    """Drafts after a commit: `out` = every token committed so far (out_tokens[0..have)),
    `prompt` = the request's prompt (the last 256 are used)."""
    have = len(out)
    w0 = max(0, have - OB_MAX)
    ob = list(out[w0:have])
    L = len(ob)
    hist = [out[have - i] if have - i >= 0 else -1 for i in range(NG_MAXN, 0, -1)]
    P = list(prompt[-OB_MAX:])
    np_ = len(P)
    drafts = []
    maxd = 0 if nodraft else T - 1
    while len(drafts) < maxd:
        d, bn = -1, 2
        j = L - 1
        while j >= 1 and bn < 8:
            m = 0
            while m < 8 and j - 1 - m >= 0 and ob[j - 1 - m] == ob[L - 1 - m]:
                m += 1
            if m > bn:
                bn, d = m, ob[j]
            j -= 1
        if d < 0:
            d = ng_next(table, hist)
        if d < 0:
            pm = 0
            j = np_ - 1
            while j >= 1 and pm < 4:
                m = 0
                while m < 4 and m < L and j - 1 - m >= 0 and P[j - 1 - m] == ob[L - 1 - m]:
                    m += 1
                if m > pm:
                    pm, d = m, P[j]
                j -= 1
        if d < 0:
            break
        drafts.append(d)
        hist.append(d)
        ob.append(d)
        L += 1
        if d in eos:
            break
    return drafts


def simulate(prompt, greedy, max_new, T, eos=(151645, 151643), table=None, nodraft=False):
    """Speculative decoding of a request whose greedy continuation is `greedy`: (committed
    tokens, passes, accepted). `greedy` must run T - 1 tokens past max_new (the last pass
    may accept drafts beyond the tokens it commits; they count as accepted) unless it ends
    with a stop token."""
    out, passes, accepted = [], 0, 0
    drafts: list[int] = []
    first = True
    while True:
        c = len(out)
        m = 0
        if not first:
            while m < len(drafts) and drafts[m] == greedy[c + m]:
                m += 1
        passes += 1
        accepted += m
        stop = False
        for k in range(m + 1):
            tok = greedy[c + k]
            out.append(tok)
            if tok in eos or len(out) >= max_new:
                stop = True
                break
        if stop:
            return out, passes, accepted
        first = False
        drafts = draft(out, prompt, T, eos, table, nodraft)
