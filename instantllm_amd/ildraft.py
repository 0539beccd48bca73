"""Learned-drafter tables in the ILDRAFT1 format, and a writer for them.

The engine's learned drafter (`ill_load_ildraft` / `ill_set_draft_context`, the drafting
kernel `ill_ildraft_kernel`) reads a table of statistics gathered from greedy outputs of
the model. The file format is the reference's (tools/draft/ildraft.py:16-53), so tables
move between the two engines unchanged; the reference ships one such table
(tools/draft/ildraft-q4.bin). This module builds a table from a list of training requests
{"prompt": text, "pids": prompt ids, "y": output ids (the stop token included when the
output stopped)} and the scorer's weights.

What the table holds (each item is a section of the format):
  * continuations: for every context of 1..max_order tokens of TAIL + y, how often it
    occurred and its most frequent next tokens (count desc, token asc; at most
    nexts_kept); contexts of 3 or more tokens seen fewer than min_count_long times are
    left out (NGKY / NGVL / NGNX);
  * a word index over the prompts (a word is a run of [a-z0-9] in the ASCII-lowercased
    UTF-8 text): per word its inverse document frequency ln((D + 1) / (df + 0.5)) and the
    requests that contain it, per request the Euclidean norm of its words' idf values, and
    per request its output (WDKY / WDVL / POST / DNRM / SQOF / SQTK);
  * copy rates: per prompt token, the share of the requests holding it whose output holds
    it too, as (copied + 0.5) / (seen + 2); per previous output token, and per previous
    pair, the share of next output tokens that occur in the prompt, as
    (hits + 0.2) / (n + 2) (CPTK / CPC1 / CPC2);
  * prompt-word associations (when enabled): per word the output tokens whose lift
    P(t in y | w in prompt) / P(t in y) is at least assoc_min_lift over at least
    assoc_min_requests requests, as ln(lift), best first (ASWK / ASWV / ASTK);
  * per-token flags (backtick count capped at 7, bit 3 = a newline byte) (TFLS);
  * the scorer: W1[H][53], b1[H], W2[H], b2, WL[53] (MLP0).
"""
from __future__ import annotations

import math
import re
import struct
from collections import Counter, defaultdict
from dataclasses import dataclass

import numpy as np

TAIL = (151645, 198, 151644, 77091, 198)   # "<|im_end|>\n<|im_start|>assistant\n"
NF = 53                                    # features per candidate
FLAG_ASSOC = 1
VOCAB = 151936
FIRST_SPECIAL = 151643                     # token ids from here on never carry flags
MAGIC = b"ILDRAFT1"


# ---- keys -------------------------------------------------------------------------------

def fnv1a64(data: bytes) -> int:
    """64-bit FNV-1a of a byte string."""
    h = 0xCBF29CE484222325
    for byte in data:
        h = ((h ^ byte) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def ctx_key(ctx) -> int:
    """Key of an n-gram context: FNV-1a over the order byte, then each token as u32 LE."""
    return fnv1a64(struct.pack(f"<B{len(ctx)}I", len(ctx), *ctx))


_WORD_RUN = re.compile(rb"[a-z0-9]+")


def prompt_words(text: str) -> list[bytes]:
    """Distinct runs of [a-z0-9] of the ASCII-lowercased UTF-8 text, first appearance first."""
    return list(dict.fromkeys(_WORD_RUN.findall(text.encode("utf-8").lower())))


# ---- configuration ----------------------------------------------------------------------

@dataclass(frozen=True)
class TableSpec:
    """What to gather, and the header values the drafter reads back."""
    max_order: int = 6            # header N: longest context
    nexts_kept: int = 6           # header M: next tokens kept per context (<= 7)
    neighbours: int = 16          # header KNB: neighbour requests the drafter consults
    max_suffix: int = 12          # header MAXM: longest suffix match
    hidden: int = 16              # header H: scorer hidden units
    min_count_long: int = 1       # header minc_hi
    associations: bool = True     # header flags bit 0
    assoc_min_requests: int = 3
    assoc_min_lift: float = 2.0
    assoc_top: int = 4            # header as_top
    edit_neighbours: int = 4      # header edit_E (the edited-neighbour option; no engine runs it)
    max_doc_share: float = 1.0    # words in more than this share of the requests are not indexed
    pair_min_count: int = 1       # CPC2 keeps pairs seen at least this often

    @property
    def flags(self) -> int:
        return FLAG_ASSOC if self.associations else 0


def random_scorer(H: int, seed: int = 0, emphasis: dict | None = None) -> dict:
    """Scorer weights: small random W1/b1/W2 plus a linear part WL, with optional extra
    weight on named feature indices (emphasis {index: weight})."""
    rng = np.random.default_rng(seed)
    W = {"W1": rng.normal(0, 0.3, (H, NF)).astype(np.float32),
         "b1": rng.normal(0, 0.1, H).astype(np.float32),
         "W2": rng.normal(0, 0.3, H).astype(np.float32),
         "b2": np.float32(rng.normal(0, 0.1)),
         "WL": rng.normal(0, 0.2, NF).astype(np.float32)}
    for i, v in (emphasis or {}).items():
        W["WL"][i] += np.float32(v)
    return W


# ---- record types of the sections (all little-endian) -------------------------------------

_U32 = np.dtype("<u4")
_U64 = np.dtype("<u8")
_F32 = np.dtype("<f4")
_NGVL = np.dtype([("total", "<u4"), ("first_n", "<u4")])
_TOKCOUNT = np.dtype([("token", "<u4"), ("count", "<u4")])
_WDVL = np.dtype([("idf", "<f4"), ("first", "<u4"), ("n", "<u4")])
_TOKRATE = np.dtype([("token", "<u4"), ("rate", "<f4")])
_PAIRRATE = np.dtype([("key", "<u8"), ("rate", "<f4"), ("zero", "<u4")])
_RANGE = np.dtype([("first", "<u4"), ("n", "<u4")])
_TOKFLAGS = np.dtype([("token", "<u4"), ("flags", "<u4")])


def _records(dtype, rows) -> np.ndarray:
    return np.array([tuple(r) for r in rows], dtype=dtype) if rows else np.zeros(0, dtype)


def _unique_keys(keys, what: str) -> None:
    if len(set(keys)) != len(keys):
        raise ValueError(f"{what} key collision")


# ---- statistics -----------------------------------------------------------------------------

class _Requests:
    """The training requests as the statistics read them."""

    def __init__(self, recs):
        self.count = len(recs)
        self.words = [prompt_words(r["prompt"]) for r in recs]
        self.prompt_sets = [frozenset(int(t) for t in r["pids"]) for r in recs]
        self.outputs = [[int(t) for t in r["y"]] for r in recs]
        # each output after the assistant tail, and where its own tokens start
        self.streams = [list(TAIL) + y for y in self.outputs]
        self.start = len(TAIL)


def _continuations(req: _Requests, spec: TableSpec):
    """[(key, total, [(token, count)...])] ascending by key."""
    follow: dict[tuple, Counter] = defaultdict(Counter)
    for s in req.streams:
        for n in range(1, spec.max_order + 1):
            for i in range(max(req.start, n), len(s)):
                follow[tuple(s[i - n:i])][s[i]] += 1
    table = []
    for ctx, nxt in follow.items():
        total = sum(nxt.values())
        if len(ctx) >= 3 and total < spec.min_count_long:
            continue
        best = sorted(nxt.items(), key=lambda tc: (-tc[1], tc[0]))[: spec.nexts_kept]
        table.append((ctx_key(ctx), total, best))
    table.sort(key=lambda e: e[0])
    _unique_keys([e[0] for e in table], "n-gram")
    return table


def _word_index(req: _Requests, spec: TableSpec):
    """({word: (idf, [request ids])}, [norm per request])."""
    holders: dict[bytes, list[int]] = defaultdict(list)
    for j, ws in enumerate(req.words):
        for w in ws:
            holders[w].append(j)
    D = req.count
    index = {w: (math.log((D + 1) / (len(js) + 0.5)), js) for w, js in holders.items() if len(js) <= spec.max_doc_share * D}
    norms = []
    for ws in req.words:
        sq = 0.0
        for w in ws:
            if w in index:
                sq += index[w][0] ** 2
        norms.append(math.sqrt(sq) or 1.0)
    return index, norms


def _copy_rates(req: _Requests, spec: TableSpec):
    """(per prompt token, per previous token, per previous pair) rates."""
    held, kept = Counter(), Counter()
    for ps, y in zip(req.prompt_sets, req.outputs):
        ys = set(y)
        held.update(ps)
        kept.update(t for t in ps if t in ys)
    token_rate = {t: (kept[t] + 0.5) / (held[t] + 2.0) for t in held}
    after1, after2 = defaultdict(lambda: [0, 0]), defaultdict(lambda: [0, 0])
    for ps, s in zip(req.prompt_sets, req.streams):
        for i in range(req.start, len(s)):
            hit = int(s[i] in ps)
            for acc in (after1[s[i - 1]], after2[(s[i - 2], s[i - 1])]):
                acc[0] += hit
                acc[1] += 1
    prev_rate = {t: (h + 0.2) / (n + 2.0) for t, (h, n) in after1.items()}
    pair_rate = {p: (h + 0.2) / (n + 2.0) for p, (h, n) in after2.items() if n >= spec.pair_min_count}
    return token_rate, prev_rate, pair_rate


def _associations(req: _Requests, spec: TableSpec):
    """{word: [(token, ln lift)...] best first}."""
    D = req.count
    with_word, with_token, both = Counter(), Counter(), Counter()
    for ws, y in zip(req.words, req.outputs):
        ys = set(y)
        with_token.update(ys)
        with_word.update(ws)
        both.update((w, t) for w in ws for t in ys)
    out: dict[bytes, list] = defaultdict(list)
    for (w, t), c in both.items():
        if c < spec.assoc_min_requests:
            continue
        lift = (c / with_word[w]) / (with_token[t] / D)
        if lift >= spec.assoc_min_lift:
            out[w].append((t, math.log(lift)))
    return {w: sorted(v, key=lambda e: (-e[1], e[0])) for w, v in out.items()}


# ---- layout ----------------------------------------------------------------------------------

class _TableFile:
    """Sections in order, each 8-byte aligned after the 64-byte header and the directory of
    {tag, count, offset} entries (16 bytes each)."""

    def __init__(self):
        self.sections: list[tuple[bytes, int, bytes]] = []

    def add(self, tag: bytes, arr: np.ndarray) -> None:
        self.sections.append((tag, len(arr), arr.tobytes()))

    def bytes(self, header: tuple) -> bytes:
        head = struct.pack("<8sII12I", MAGIC, 1, len(self.sections), *header)
        at = -(-(len(head) + 16 * len(self.sections)) // 8) * 8
        directory, body = [], []
        for tag, count, data in self.sections:
            directory.append(struct.pack("<4sIQ", tag, count, at))
            padded = data + bytes(-len(data) % 8)
            body.append(padded)
            at += len(padded)
        front = head + b"".join(directory)
        return front + bytes(-len(front) % 8) + b"".join(body)


def build(recs, spec: TableSpec, scorer: dict, tok_flags: dict | None = None) -> bytes:
    """The ILDRAFT1 table of `recs` (list of {"prompt", "pids", "y"}) as bytes."""
    if spec.nexts_kept > 7 or spec.max_order > 6:
        raise ValueError("at most 7 next tokens per context and contexts of at most 6 tokens")
    req = _Requests(recs)
    f = _TableFile()

    cont = _continuations(req, spec)
    spans = np.cumsum([0] + [len(best) for _, _, best in cont])
    f.add(b"NGKY", np.array([k for k, _, _ in cont], _U64))
    f.add(b"NGVL", _records(_NGVL, [(total, (int(spans[i]) << 3) | len(best)) for i, (_, total, best) in enumerate(cont)]))
    f.add(b"NGNX", _records(_TOKCOUNT, [tc for _, _, best in cont for tc in best]))

    index, norms = _word_index(req, spec)
    by_key = sorted((fnv1a64(w), w) for w in index)
    _unique_keys([k for k, _ in by_key], "word")
    post_spans = np.cumsum([0] + [len(index[w][1]) for _, w in by_key])
    f.add(b"WDKY", np.array([k for k, _ in by_key], _U64))
    f.add(b"WDVL", _records(_WDVL, [(index[w][0], int(post_spans[i]), len(index[w][1])) for i, (_, w) in enumerate(by_key)]))
    f.add(b"POST", np.array([j for _, w in by_key for j in index[w][1]], _U32))
    f.add(b"DNRM", np.array(norms, _F32))
    f.add(b"SQOF", np.cumsum([0] + [len(y) for y in req.outputs]).astype(_U32))
    f.add(b"SQTK", np.array([t for y in req.outputs for t in y], _U32))

    token_rate, prev_rate, pair_rate = _copy_rates(req, spec)
    f.add(b"CPTK", _records(_TOKRATE, sorted(token_rate.items())))
    f.add(b"CPC1", _records(_TOKRATE, sorted(prev_rate.items())))
    f.add(b"CPC2", _records(_PAIRRATE, sorted(((a << 32) | b, r, 0) for (a, b), r in pair_rate.items())))

    if spec.associations:
        assoc = _associations(req, spec)
        words = sorted((fnv1a64(w), w) for w in assoc)
        _unique_keys([k for k, _ in words], "association word")
        lists = [assoc[w] for _, w in words]
        starts = np.cumsum([0] + [len(v) for v in lists])
        f.add(b"ASWK", np.array([k for k, _ in words], _U64))
        f.add(b"ASWV", _records(_RANGE, [(int(starts[i]), len(v)) for i, v in enumerate(lists)]))
        f.add(b"ASTK", _records(_TOKRATE, [e for v in lists for e in v]))

    flagged = sorted((int(t), int(v)) for t, v in (tok_flags or {}).items() if v and 0 <= t < FIRST_SPECIAL)
    f.add(b"TFLS", _records(_TOKFLAGS, flagged))

    H = len(scorer["b1"])
    mlp = np.concatenate([np.asarray(scorer[k], np.float32).reshape(-1) for k in ("W1", "b1", "W2")]
                         + [np.asarray([scorer["b2"]], np.float32), np.asarray(scorer["WL"], np.float32)])
    if mlp.size != H * NF + 2 * H + 1 + NF:
        raise ValueError("scorer weights do not match H x 53")
    f.add(b"MLP0", mlp.astype(_F32))

    header = (spec.max_order, spec.nexts_kept, spec.neighbours, spec.max_suffix, NF, H, spec.min_count_long,
              req.count, spec.flags, spec.assoc_top, spec.edit_neighbours, 0)
    return f.bytes(header)


def save(path: str, recs, spec: TableSpec, scorer: dict, tok_flags: dict | None = None) -> int:
    blob = build(recs, spec, scorer, tok_flags)
    with open(path, "wb") as fh:
        fh.write(blob)
    return len(blob)
