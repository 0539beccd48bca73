"""Learned-drafter tables in the ILDRAFT1 format, and their builder.

The engine's learned drafter (`ill_load_ildraft` / `ill_set_draft_context`, the drafting
kernel `ill_ildraft_kernel`) reads a table file built from greedy outputs of the model
(tools/draft/ildraft.py:16-53 is the format; `Tables.build` :134-227 the statistics; the
reference's shipped table is tools/draft/ildraft-q4.bin). This module writes that format
from a list of records {"prompt": text, "pids": prompt ids, "y": output ids (stop token
included when the output stopped)} and the scorer's weights.

Table contents (the format is fixed so that tables move between the engines unchanged):
  * n-gram continuations of TAIL + y, for every context of 1..N tokens: total count and the
    top M next tokens (count desc, token asc); contexts of >= 3 tokens with fewer than
    minc_hi occurrences are dropped;
  * a TF-IDF index over prompt words (runs of [a-z0-9] of the ASCII-lowercased prompt):
    idf = ln((D + 1) / (df + 0.5)), postings, per-document norms, and each document's output;
  * copy statistics: per prompt token the rate of appearing in the output
    ((copied + 0.5) / (seen + 2)), per previous token / token pair the rate of the next
    output token being a prompt token ((hits + 0.2) / (n + 2));
  * prompt-word -> output-token associations (flags & 1): ln(lift) for pairs seen in at
    least as_min requests with lift = P(t in y | w in prompt) / P(t in y) >= as_lift;
  * per-token flags (number of '`' bytes capped at 7, bit 3 = a newline byte);
  * the scorer: W1[H][53], b1[H], W2[H], b2, WL[53].
"""
from __future__ import annotations

import math
import re
import struct
from collections import defaultdict
from dataclasses import dataclass

import numpy as np

TAIL = (151645, 198, 151644, 77091, 198)   # "<|im_end|>\n<|im_start|>assistant\n"
NF = 53                                    # features per candidate
FLAG_ASSOC = 1
VOCAB = 151936

_FNV_OFF = 0xCBF29CE484222325
_FNV_PRIME = 0x100000001B3
_M64 = (1 << 64) - 1
_WORD = re.compile(rb"[a-z0-9]+")


def fnv1a64(b: bytes) -> int:
    h = _FNV_OFF
    for x in b:
        h = ((h ^ x) * _FNV_PRIME) & _M64
    return h


def ctx_key(ctx) -> int:
    """Key of an n-gram context: FNV-1a over the order byte, then each token as u32 LE."""
    return fnv1a64(bytes([len(ctx)]) + struct.pack(f"<{len(ctx)}I", *ctx))


def prompt_words(text: str) -> list[bytes]:
    """Distinct runs of [a-z0-9] of the ASCII-lowercased UTF-8 text, first appearance first."""
    out, seen = [], set()
    for w in _WORD.findall(text.encode("utf-8").lower()):
        if w not in seen:
            seen.add(w)
            out.append(w)
    return out


@dataclass
class DraftConfig:
    N: int = 6          # longest n-gram context
    M: int = 6          # next tokens kept per context
    KNB: int = 16       # neighbours per request
    MAXM: int = 12      # longest suffix match
    H: int = 16         # scorer hidden units
    minc_hi: int = 1
    flags: int = FLAG_ASSOC
    as_min: int = 3
    as_lift: float = 2.0
    as_top: int = 4
    edit_E: int = 4
    max_df: float = 1.0
    cc2_min: int = 1


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


def build(recs, cfg: DraftConfig, scorer: dict, tok_flags: dict | None = None) -> bytes:
    """The ILDRAFT1 table of `recs` (list of {"prompt", "pids", "y"}) as bytes."""
    assert cfg.M <= 7 and cfg.N <= 6
    # ---- n-gram continuations of TAIL + y ----
    counts: dict = defaultdict(lambda: defaultdict(int))
    for r in recs:
        s = list(TAIL) + [int(t) for t in r["y"]]
        for i in range(len(TAIL), len(s)):
            for n in range(1, cfg.N + 1):
                if i - n < 0:
                    break
                counts[tuple(s[i - n:i])][s[i]] += 1
    ng = []
    for ctx, d in counts.items():
        tot = sum(d.values())
        if len(ctx) >= 3 and tot < cfg.minc_hi:
            continue
        top = sorted(d.items(), key=lambda kv: (-kv[1], kv[0]))[:cfg.M]
        ng.append((ctx_key(ctx), tot, top))
    ng.sort(key=lambda e: e[0])
    assert all(a[0] != b[0] for a, b in zip(ng, ng[1:])), "n-gram key collision"
    # ---- TF-IDF over prompt words ----
    D = len(recs)
    docs = [prompt_words(r["prompt"]) for r in recs]
    df: dict = defaultdict(int)
    post: dict = defaultdict(list)
    for j, ws in enumerate(docs):
        for w in ws:
            df[w] += 1
            post[w].append(j)
    vocab = {w: (math.log((D + 1) / (c + 0.5)), post[w]) for w, c in df.items() if c <= cfg.max_df * D}
    norms = [math.sqrt(sum(vocab[w][0] ** 2 for w in ws if w in vocab)) or 1.0 for ws in docs]
    # ---- copy statistics ----
    seen: dict = defaultdict(int)
    copied: dict = defaultdict(int)
    c1: dict = defaultdict(lambda: [0, 0])
    c2: dict = defaultdict(lambda: [0, 0])
    for r in recs:
        ps, ys = set(int(t) for t in r["pids"]), set(int(t) for t in r["y"])
        for x in ps:
            seen[x] += 1
            copied[x] += x in ys
        s = list(TAIL) + [int(t) for t in r["y"]]
        for i in range(len(TAIL), len(s)):
            hit = 1 if s[i] in ps else 0
            for e in (c1[s[i - 1]], c2[(s[i - 2], s[i - 1])]):
                e[0] += hit
                e[1] += 1
    prop = {x: (copied[x] + 0.5) / (seen[x] + 2.0) for x in seen}
    cc1 = {k: (v[0] + 0.2) / (v[1] + 2.0) for k, v in c1.items()}
    cc2 = {k: (v[0] + 0.2) / (v[1] + 2.0) for k, v in c2.items() if v[1] >= cfg.cc2_min}
    # ---- associations ----
    assoc = {}
    if cfg.flags & FLAG_ASSOC:
        cw: dict = defaultdict(int)
        ct: dict = defaultdict(int)
        cwt: dict = defaultdict(int)
        for r, ws in zip(recs, docs):
            ys = set(int(t) for t in r["y"])
            for x in ys:
                ct[x] += 1
            for w in ws:
                cw[w] += 1
                for x in ys:
                    cwt[(w, x)] += 1
        pairs: dict = defaultdict(list)
        for (w, x), c in cwt.items():
            if c >= cfg.as_min:
                lift = (c / cw[w]) / (ct[x] / D)
                if lift >= cfg.as_lift:
                    pairs[w].append((x, math.log(lift)))
        assoc = {w: sorted(v, key=lambda e: (-e[1], e[0])) for w, v in pairs.items()}

    # ---- sections ----
    secs = []
    vl, nx = bytearray(), bytearray()
    first = 0
    for _, tot, top in ng:
        vl += struct.pack("<II", tot, (first << 3) | len(top))
        for tok, c in top:
            nx += struct.pack("<II", tok, c)
        first += len(top)
    secs += [(b"NGKY", len(ng), struct.pack(f"<{len(ng)}Q", *[e[0] for e in ng])),
             (b"NGVL", len(ng), bytes(vl)), (b"NGNX", first, bytes(nx))]
    words = sorted((fnv1a64(w), w) for w in vocab)
    assert all(a[0] != b[0] for a, b in zip(words, words[1:])), "word key collision"
    wv, po = bytearray(), []
    for _, w in words:
        idf, plist = vocab[w]
        wv += struct.pack("<fII", idf, len(po), len(plist))
        po += plist
    secs += [(b"WDKY", len(words), struct.pack(f"<{len(words)}Q", *[h for h, _ in words])),
             (b"WDVL", len(words), bytes(wv)),
             (b"POST", len(po), struct.pack(f"<{len(po)}I", *po)),
             (b"DNRM", D, struct.pack(f"<{D}f", *norms))]
    offs, toks = [0], []
    for r in recs:
        toks += [int(t) for t in r["y"]]
        offs.append(len(toks))
    secs += [(b"SQOF", len(offs), struct.pack(f"<{len(offs)}I", *offs)),
             (b"SQTK", len(toks), struct.pack(f"<{len(toks)}I", *toks))]
    secs.append((b"CPTK", len(prop), b"".join(struct.pack("<If", k, v) for k, v in sorted(prop.items()))))
    secs.append((b"CPC1", len(cc1), b"".join(struct.pack("<If", k, v) for k, v in sorted(cc1.items()))))
    k2 = sorted(((a << 32) | b, v) for (a, b), v in cc2.items())
    secs.append((b"CPC2", len(k2), b"".join(struct.pack("<QfI", k, v, 0) for k, v in k2)))
    if cfg.flags & FLAG_ASSOC:
        aw = sorted((fnv1a64(w), w) for w in assoc)
        assert all(a[0] != b[0] for a, b in zip(aw, aw[1:])), "association word key collision"
        av, at = bytearray(), bytearray()
        first = 0
        for _, w in aw:
            lst = assoc[w]
            av += struct.pack("<II", first, len(lst))
            for tok, ll in lst:
                at += struct.pack("<If", tok, ll)
            first += len(lst)
        secs += [(b"ASWK", len(aw), struct.pack(f"<{len(aw)}Q", *[h for h, _ in aw])),
                 (b"ASWV", len(aw), bytes(av)), (b"ASTK", first, bytes(at))]
    tf = sorted((int(t), int(v)) for t, v in (tok_flags or {}).items() if v and 0 <= t < 151643)
    secs.append((b"TFLS", len(tf), b"".join(struct.pack("<II", t, v) for t, v in tf)))
    W = scorer
    H = len(W["b1"])
    flat = np.concatenate([np.asarray(W["W1"], np.float32).reshape(-1), np.asarray(W["b1"], np.float32),
                           np.asarray(W["W2"], np.float32), np.asarray([W["b2"]], np.float32),
                           np.asarray(W["WL"], np.float32)])
    assert flat.size == H * NF + 2 * H + 1 + NF
    secs.append((b"MLP0", flat.size, flat.tobytes()))

    hdr_len = 64 + 16 * len(secs)
    off = (hdr_len + 7) // 8 * 8
    dirs, body = bytearray(), bytearray()
    for tag, cnt, data in secs:
        dirs += struct.pack("<4sIQ", tag, cnt, off)
        pad = (-len(data)) % 8
        body += data + b"\0" * pad
        off += len(data) + pad
    hdr = struct.pack("<8sII" + "I" * 12, b"ILDRAFT1", 1, len(secs), cfg.N, cfg.M, cfg.KNB, cfg.MAXM, NF, H,
                      cfg.minc_hi, D, cfg.flags, cfg.as_top, cfg.edit_E, 0)
    blob = bytearray(hdr + dirs)
    blob += b"\0" * ((-len(blob)) % 8)
    return bytes(blob + body)


def save(path: str, recs, cfg: DraftConfig, scorer: dict, tok_flags: dict | None = None) -> int:
    blob = build(recs, cfg, scorer, tok_flags)
    with open(path, "wb") as f:
        f.write(blob)
    return len(blob)
