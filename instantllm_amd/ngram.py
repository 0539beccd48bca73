"""n-gram draft tables for speculative decoding, in the reference's NGramTable layout
(Sources/Engine/NGram.swift:1-59; lookup NGEntry / ng_next, Shaders.swift:56-86).

For every context of the last 1..6 generated tokens (padded with -1 before the output
starts) the table stores the most frequent next token (ties: the lowest id), its count and
the context's total, in 2^20 open-addressed 16-byte slots {u64 key, i32 next, u16 count,
u16 total} placed by linear probing (at most 16 probes) from slot (key >> 12) mod 2^20.
The key is NGramTable.key's FNV-style hash, so tables built by the reference load as they
are. Contexts are inserted in ascending key order (the reference inserts in Swift dictionary
order, so colliding contexts may sit in other slots; every lookup still finds its key).

`Engine.load_ngram(build(seqs))` hands a table to the device drafter.
"""
from __future__ import annotations

from collections import defaultdict

import numpy as np

SLOTS = 1 << 20
MAXN = 6
ENTRY = np.dtype([("key", "<u8"), ("next", "<i4"), ("count", "<u2"), ("total", "<u2")])
M64 = (1 << 64) - 1


def key(ctx) -> int:
    h = 0xCBF29CE484222325 ^ len(ctx)
    for t in ctx:
        h ^= ((int(t) & 0xFFFFFFFF) + 0x9E3779B97F4A7C15) & M64
        h = (h * 0x100000001B3) & M64
        h ^= h >> 29
    return h | 1


def build(seqs) -> np.ndarray:
    """Table [SLOTS] of ENTRY from token sequences (each ending with its stop token)."""
    counts: dict[int, dict[int, int]] = defaultdict(lambda: defaultdict(int))
    for seq in seqs:
        s = [-1] * MAXN + [int(t) for t in seq]
        for i in range(MAXN, len(s)):
            for n in range(1, MAXN + 1):
                counts[key(s[i - n:i])][s[i]] += 1
    table = np.zeros(SLOTS, ENTRY)
    for k in sorted(counts):
        nexts = counts[k]
        total = sum(nexts.values())
        tok, c = min(nexts.items(), key=lambda kv: (-kv[1], kv[0]))
        slot = (k >> 12) & (SLOTS - 1)
        for _ in range(16):
            if table["key"][slot] == 0:
                table[slot] = (k, tok, min(c, 65535), min(total, 65535))
                break
            slot = (slot + 1) & (SLOTS - 1)
    return table
