"""Synthetic request corpus and tokenizer stand-in for the learned-drafter tests.

Requests come in families: each family has a prompt template (words) and an output
template (token ids) with slots that copy prompt words, their space variants (the id that
`mock_encode(" " + word)` gives) or family-specific tokens. Outputs stay under 76 tokens
(TAIL + output fits the engine's 80-token neighbour sequences) and prompts under 40 ids.
"""
from __future__ import annotations

import numpy as np

VOCAB = 4096
STOP = 151645


def _fnv(b: bytes) -> int:
    h = 0xCBF29CE484222325
    for x in b:
        h = ((h ^ x) * 0x100000001B3) & ((1 << 64) - 1)
    return h


def tok_id(word: str) -> int:
    """The stand-in tokenizer's id of a prompt word."""
    return 100 + _fnv(word.encode()) % (VOCAB - 200)


def mock_encode(text: str) -> list[int]:
    """The stand-in tokenizer: one id per text (a leading space gives a different id)."""
    return [100 + _fnv(b"enc:" + text.encode()) % (VOCAB - 200)]


def _words(rng, n, lo=3, hi=8):
    letters = np.array(list("abcdefghijklmnopqrstuvwxyz"))
    return ["".join(rng.choice(letters, rng.integers(lo, hi + 1))) for _ in range(n)]


class Corpus:
    def __init__(self, seed=0, families=24):
        rng = np.random.default_rng(seed)
        self.rng = rng
        self.vocab_words = _words(rng, 240) + [f"{w}_{v}.py" for w, v in zip(_words(rng, 12), range(12))] \
            + [f"src/{w}" for w in _words(rng, 12)] + [f"v{i}.{i + 1}" for i in range(6)]
        self.fam = []
        for _ in range(families):
            tmpl = list(rng.choice(self.vocab_words[:240], rng.integers(4, 8), replace=False))
            body = [int(x) for x in rng.integers(100, VOCAB, rng.integers(12, 40))]
            # output = body pieces with slots: -1 copy a slot word's id, -2 its space variant
            out = []
            for k, t in enumerate(body):
                out.append(t)
                if k % 5 == 2:
                    out.append(-1 if rng.random() < 0.6 else -2)
            self.fam.append((tmpl, out, bool(rng.random() < 0.7)))
        self.flags = {int(t): int(rng.integers(1, 16)) for t in rng.integers(100, VOCAB, 60)}

    def request(self, f, rng=None):
        rng = rng or self.rng
        tmpl, out, stops = self.fam[f]
        slots = list(rng.choice(self.vocab_words, rng.integers(2, 5), replace=False))
        words = tmpl + slots
        if rng.random() < 0.3:
            rng.shuffle(words)
        text = " ".join(w.capitalize() if rng.random() < 0.2 else w for w in words)
        if rng.random() < 0.5:
            text += "?"
        pids = [tok_id(w) for w in words]
        y, si = [], 0
        for t in out:
            if t >= 0:
                y.append(t if rng.random() > 0.05 else int(rng.integers(100, VOCAB)))
            else:
                w = slots[si % len(slots)]
                si += 1
                y.append(tok_id(w) if t == -1 else mock_encode(" " + w)[0])
        y = y[:75]
        if stops and len(y) < 75:
            y.append(STOP)
        return {"prompt": text, "pids": pids, "y": y}

    def records(self, n):
        return [self.request(int(self.rng.integers(0, len(self.fam)))) for _ in range(n)]
