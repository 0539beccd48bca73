"""Tree-verify semantics (oracle).

Tree layout (`Sources/Engine/Shaders.swift:23-30`): ints [n, depth[16], parent[16],
tok[16], anc[16]]; row 0 is the last committed token, row i a draft whose parent row is
parent[i] < i; anc[i] has bit j set for every row j on its path (itself included). Row i
occupies KV slot pos + i, is rotated as position pos + depth[i] and attends to the context
[0, pos) plus its ancestors (`Shaders.swift:893-950`, `:2001`).

Accept rule (`Shaders.swift:305-320`): from the root, repeatedly take the lowest-index
child whose token equals the current row's argmax. Commit (`:322-333`): g[root], then
g[path[0]], ... stopping after a stop token or when maxsteps is reached. KV compaction
(`:351-365`): the accepted row path[k-1] moves from slot pos + path[k-1] to pos + k.
"""
from __future__ import annotations

import numpy as np

from .qwen import Model, KV, rope_cos_sin

TR_DEPTH, TR_PARENT, TR_TOK, TR_ANC, TR_INTS = 1, 17, 33, 49, 65


def make_tree(parent: list[int], tok: list[int]) -> np.ndarray:
    """Build the 65-int tree buffer from parent indices (parent[0] ignored)."""
    n = len(tok)
    assert 1 <= n <= 16 and len(parent) == n
    t = np.zeros(TR_INTS, np.int32)
    t[0] = n
    depth = [0] * n
    anc = [1] * n
    for i in range(1, n):
        p = parent[i]
        assert 0 <= p < i
        depth[i] = depth[p] + 1
        anc[i] = anc[p] | (1 << i)
    t[TR_DEPTH:TR_DEPTH + n] = depth
    t[TR_PARENT:TR_PARENT + n] = [0] + list(parent[1:])
    t[TR_TOK:TR_TOK + n] = tok
    t[TR_ANC:TR_ANC + n] = anc
    return t


def random_tree(rng: np.random.Generator, n: int, vocab: int) -> np.ndarray:
    """Config 3 shape: parent[i] uniform over 0..i-1, tokens uniform in [0, vocab)."""
    parent = [0] + [int(rng.integers(0, i)) for i in range(1, n)]
    tok = [int(t) for t in rng.integers(0, vocab, size=n)]
    return make_tree(parent, tok)


def paths(tree: np.ndarray) -> list[list[int]]:
    """Root-to-leaf row paths."""
    n = int(tree[0])
    par = tree[TR_PARENT:TR_PARENT + n]
    kids = {i: [j for j in range(1, n) if par[j] == i] for i in range(n)}
    out = []
    for i in range(n):
        if not kids[i]:
            p, r = [], i
            while True:
                p.append(r)
                if r == 0:
                    break
                r = int(par[r])
            out.append(p[::-1])
    return out


def tree_logits(m: Model, cache: KV, tree: np.ndarray) -> np.ndarray:
    """Logits [n, V] of every tree row in one wide pass at positions cache.len + depth.
    Writes the rows' K/V at slots cache.len + i and leaves cache.len unchanged."""
    n = int(tree[0])
    pos = cache.len
    depth = tree[TR_DEPTH:TR_DEPTH + n].astype(np.int64)
    anc = tree[TR_ANC:TR_ANC + n].astype(np.int64)
    tok = tree[TR_TOK:TR_TOK + n].astype(np.int64)
    cos, sin = rope_cos_sin(pos + depth, m.dtype)
    slots = pos + np.arange(n)
    K_slots = np.arange(pos + n)
    allowed = np.ones((n, pos + n), bool)
    for i in range(n):
        for j in range(n):
            allowed[i, pos + j] = bool((anc[i] >> j) & 1)
    x = m.embed[tok]
    for li in range(len(m.layers)):
        x = m.layer(li, x, cos, sin, slots, K_slots, allowed, cache)
    return m.logits(x)


def accept(tree: np.ndarray, g: list[int]) -> list[int]:
    """Accepted row path (excluding the root) for per-row argmaxes g."""
    n = int(tree[0])
    par = tree[TR_PARENT:TR_PARENT + n]
    tok = tree[TR_TOK:TR_TOK + n]
    path, cur = [], 0
    while True:
        c = next((i for i in range(1, n) if par[i] == cur and tok[i] == g[cur]), -1)
        if c < 0:
            return path
        path.append(c)
        cur = c


def commit_tokens(tree: np.ndarray, g: list[int], step: int, maxsteps: int, eos=(151645, 151643)):
    """Tokens committed by one tree pass, the stop flag and the accepted path."""
    path = accept(tree, g)
    out = []
    stop = False
    for i in range(len(path) + 1):
        t = g[0] if i == 0 else g[path[i - 1]]
        out.append(int(t))
        step += 1
        if t in eos or step >= maxsteps:
            stop = True
            break
    return out, stop, path


def chain_accept(drafts: list[int], g: list[int]) -> int:
    """Accepted drafts of a chain pass: longest prefix with drafts[m] == g[m]
    (`Shaders.swift:321`)."""
    m = 0
    while m < len(g) - 1 and m < len(drafts) and drafts[m] == g[m]:
        m += 1
    return m
