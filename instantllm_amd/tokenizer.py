"""Qwen2 byte-level BPE tokenizer: the reference's `Sources/Tokenizer` (Tokenizer.swift,
Core.swift, Compile.swift, UnicodeData.swift) for the Linux host.

Two halves, like the reference's `Tokenizer.compile` / `Tokenizer(path:)`:

- `compile(tokenizer_json, out)` (Compile.swift:14-371) checks that a Hugging Face
  tokenizer.json is the Qwen2 pipeline (NFC normalizer, the Qwen2 split regex + byte-level
  pre-tokenizer, byte-level BPE, byte-level decoder, added tokens matched on the raw text)
  and writes an ILTK1 file: token bytes, a hash table of the tokens a whole pre-tokenizer
  piece may map to directly, the merge table, the added tokens and the Unicode tables the
  encoder needs.
- `Tokenizer(path)` maps that file in libillhip.so (`ill_tok_open`) and encodes / decodes
  natively (`ill_tok_encode`, `ill_tok_encode_chat`, `ill_tok_decode`: Tokenizer.swift:
  150-331); `TextStream` is the reference's incremental detokenizer (:337-441).

The Unicode tables are taken from Hugging Face `tokenizers` itself, which the reference
treats as the definition (tools/tokenizer_unicode.py:1-20): its split regex runs on
Oniguruma and its NFC on the `unicode-normalization-alignments` crate, each with its own
Unicode version, different from Python's `unicodedata`. `unicode_tables()` asks the
installed `tokenizers` for every code point: the regex classes \\p{L}, \\p{N}, \\s, the
letters the case-insensitive contractions accept, each code point's canonical decomposition
(its NFD), which combining marks the NFC crate reorders (canonical classes from
`unicodedata`, kept only where the crate reorders them), and the primary compositions (pairs
that its NFC composes). Compiling therefore needs `tokenizers`; encoding does not.

ILTK1 layout (little endian; header of 64 u64 words, then 8-byte aligned sections):
  word 0 magic, 1 file size, 2 n_total (ids), 3 n_vocab, 4 n_merges, 5 n_added,
  6 longest vocab token (bytes), 7 log2 token slots, 8 log2 merge slots,
  9-11 ids of <|im_start|>, <|im_end|>, <|endoftext|> (-1: absent), 12 Unicode blocks,
  13 decompositions, 14 decomposition code points, 15 compositions, 16 ignore_merges;
  words 20-33 section offsets:
  20 tok_off u32[n_total + 1]   21 tok_bytes (decoded bytes of each id)
  22 byte_tok i32[256]          23 tok_slots u32[2^b] (id + 1 of a direct token; 0 empty)
  24 merge_slots {u64 key = left << 32 | right (~0 empty), u32 rank, u32 merged id}[2^b]
  25 added u32[3 n_added] (id, offset, length into 26)   26 added bytes (UTF-8 content)
  27 uni_top u16[0x1100] (block of each 256 code points)   28 uni_blocks u16[blocks][256]
  29 decomp_keys u32[] (sorted)  30 decomp_vals u32[] (offset << 8 | length into 31)
  31 decomp_data u32[]           32 comp_keys u64[] (sorted, first << 21 | second)
  33 comp_vals u32[]
  Unicode property (u16): bits 0-2 split class (0 letter, 1 number, 2 other, 3 other
  whitespace, 4 space, 5 CR/LF), bit 3 the code point may change under NFC, bits 4-7 the
  contraction letters after an apostrophe (s t m d; r v; e; l), bits 8-15 canonical class.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct
import sys
from pathlib import Path

import numpy as np

QWEN2_SPLIT = r"""(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+"""
CHAT_TEMPLATE = "<|im_start|>system\n{s}<|im_end|>\n<|im_start|>user\n{u}<|im_end|>\n<|im_start|>assistant\n"

MAGIC = 0x31304B544C49    # "ILTK01"
HDR_WORDS = 64
CL, CN, CO, CWS, CSP, CNL = 0, 1, 2, 3, 4, 5
F_NFC, F_C1, F_RV, F_E, F_LL = 1 << 3, 1 << 4, 1 << 5, 1 << 6, 1 << 7
NCP = 0x110000
HANGUL_V = range(0x1161, 0x1176)
HANGUL_T = range(0x11A8, 0x11C3)
S_BASE, S_COUNT = 0xAC00, 11172


def byte_alphabet() -> dict[int, str]:
    """The byte-level alphabet of GPT-2 style BPE (HF ByteLevel): printable Latin-1 bytes
    stand for themselves, the other 68 bytes for code points 256, 257, ... in byte order."""
    keep = list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    out, k = {}, 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + k)
            k += 1
    return out


# ---- Unicode tables, from the installed Hugging Face `tokenizers` -------------------------

def _batch(norm, strs: list[str], sep: str = "\x00") -> list[str]:
    """norm.normalize_str of each string, many per call, joined by a starter that neither
    decomposes nor composes (strings holding the separator are normalized alone)."""
    out: list[str | None] = [None] * len(strs)
    idx = [i for i, s in enumerate(strs) if sep not in s]
    for k in range(0, len(idx), 20000):
        part = idx[k:k + 20000]
        res = norm.normalize_str(sep.join(strs[i] for i in part)).split(sep)
        if len(res) != len(part):
            raise RuntimeError("normalizer output does not split back into its inputs")
        for i, r in zip(part, res):
            out[i] = r
    for i, s in enumerate(strs):
        if out[i] is None:
            out[i] = norm.normalize_str(s)
    return out   # type: ignore[return-value]


def _members(rx: str, cps: np.ndarray) -> np.ndarray:
    """Code points matched by a one-character Oniguruma pattern, by splitting runs of them
    out with HF's pre-tokenizer (the pieces it keeps are the non-matching runs)."""
    from tokenizers import Regex, pre_tokenizers
    sp = pre_tokenizers.Split(Regex(rx), behavior="removed")
    hit = np.ones(len(cps), bool)
    for k in range(0, len(cps), 50000):
        chunk = cps[k:k + 50000]
        for _, (a, b) in sp.pre_tokenize_str("".join(map(chr, chunk))):
            hit[k + a:k + b] = False
    return cps[hit]


def unicode_tables():
    """(props u16[0x110000], decompositions {cp: [cps]}, compositions {(a, b): cp}) as the
    installed `tokenizers` behaves."""
    import unicodedata
    try:
        from tokenizers import normalizers
    except ImportError as e:   # pragma: no cover
        raise RuntimeError("compiling a tokenizer needs the Hugging Face `tokenizers` package") from e
    cps = np.array([c for c in range(NCP) if not 0xD800 <= c <= 0xDFFF], np.int64)
    props = np.full(NCP, CO, np.uint16)
    props[_members(r"\p{L}", cps)] = CL
    props[_members(r"\p{N}", cps)] = CN
    props[_members(r"\s", cps)] = CWS
    props[0x20] = CSP
    props[0x0A] = props[0x0D] = CNL
    for letters, flag in (("stmd", F_C1), ("rv", F_RV), ("e", F_E), ("l", F_LL)):
        for ch in letters:
            props[_members("(?i:%s)" % ch, cps)] |= flag
    nfd_n, nfc_n = normalizers.NFD(), normalizers.NFC()
    chars = [chr(c) for c in cps]
    decomp = {}
    for c, d in zip(cps.tolist(), _batch(nfd_n, chars)):
        if d != chr(c) and not S_BASE <= c < S_BASE + S_COUNT:   # Hangul: algorithmic
            decomp[c] = [ord(x) for x in d]
    # canonical classes the NFC crate knows: a mark of class < 230 moves in front of U+0301
    # (class 230), one of class >= 230 behind U+0334 (class 1)
    marks = [c for c in cps.tolist() if unicodedata.combining(chr(c))]
    lo = [c for c in marks if unicodedata.combining(chr(c)) < 230]
    hi = [c for c in marks if unicodedata.combining(chr(c)) >= 230]
    for c, r in zip(lo, _batch(nfd_n, ["a\u0301" + chr(c) for c in lo])):
        if r == "a" + chr(c) + "\u0301":
            props[c] |= unicodedata.combining(chr(c)) << 8
    for c, r in zip(hi, _batch(nfd_n, ["a" + chr(c) + "\u0334" for c in hi])):
        if r == "a\u0334" + chr(c):
            props[c] |= unicodedata.combining(chr(c)) << 8
    # primary compositions: canonical pairs that the crate's NFC composes
    pairs = []
    for c in decomp:
        d = unicodedata.decomposition(chr(c))
        if d and not d.startswith("<"):
            parts = [int(x, 16) for x in d.split()]
            if len(parts) == 2:
                pairs.append((parts[0], parts[1], c))
    comp = {}
    for (a, b, c), r in zip(pairs, _batch(nfc_n, [chr(a) + chr(b) for a, b, _ in pairs])):
        if r == chr(c):
            comp[(a, b)] = c
    # may change under NFC somewhere: NFC of the code point alone differs, a non-starter, or
    # the second element of a composition (Hangul vowels and trailing consonants included)
    alone = _batch(nfc_n, chars)
    for c, r in zip(cps.tolist(), alone):
        if r != chr(c):
            props[c] |= F_NFC
    props[(props >> 8) != 0] |= F_NFC
    for (_, b) in comp:
        props[b] |= F_NFC
    for c in list(HANGUL_V) + list(HANGUL_T):
        props[c] |= F_NFC
    return props, decomp, comp


# ---- BPE (compile time: which tokens a whole piece maps to directly) ----------------------

def _bpe(sym: list[int], merges: dict) -> list[int]:
    """Byte-pair merges of one piece, lowest rank first and leftmost among equal ranks (the
    order of HF's (rank, position) heap)."""
    sym = list(sym)
    while len(sym) > 1:
        best, bi = None, -1
        for i in range(len(sym) - 1):
            m = merges.get((sym[i], sym[i + 1]))
            if m is not None and (best is None or m[0] < best[0]):
                best, bi = m, i
        if best is None:
            break
        sym[bi:bi + 2] = [best[1]]
    return sym


def _hash_bytes(b: bytes) -> int:
    """FNV-1a 64 (the same function in ill_tok.h)."""
    h = 0xCBF29CE484222325
    for x in b:
        h = ((h ^ x) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _check_pipeline(j: dict) -> None:
    """The Qwen2 pipeline (Compile.swift checkPipeline semantics): anything else would need
    behaviour the encoder does not have."""
    def bad(what):
        raise ValueError(f"unsupported tokenizer.json: {what}")
    norm = j.get("normalizer") or {}
    if norm.get("type") != "NFC":
        bad(f"normalizer {norm.get('type')}")
    pre = j.get("pre_tokenizer") or {}
    seq = pre.get("pretokenizers", []) if pre.get("type") == "Sequence" else []
    if len(seq) != 2 or seq[0].get("type") != "Split" or seq[1].get("type") != "ByteLevel":
        bad("pre_tokenizer is not Sequence[Split, ByteLevel]")
    pat = seq[0].get("pattern", {})
    if pat.get("Regex") != QWEN2_SPLIT or seq[0].get("behavior") != "Isolated" or seq[0].get("invert"):
        bad("split regex is not Qwen2's")
    if seq[1].get("add_prefix_space") or seq[1].get("use_regex"):
        bad("ByteLevel with a prefix space or its own regex")
    m = j.get("model") or {}
    if m.get("type") != "BPE" or m.get("dropout") or m.get("continuing_subword_prefix") or m.get("end_of_word_suffix") \
            or m.get("byte_fallback"):
        bad("model is not plain byte-level BPE")
    dec = j.get("decoder") or {}
    if dec.get("type") != "ByteLevel":
        bad(f"decoder {dec.get('type')}")


def compile(tokenizer_json: str | os.PathLike, out: str | os.PathLike, tables=None) -> dict:
    """tokenizer.json -> ILTK1 file (Tokenizer.compile, Compile.swift:14-371). `tables`: the
    result of unicode_tables() to reuse. Returns a summary."""
    j = json.loads(Path(tokenizer_json).read_text(encoding="utf-8"))
    _check_pipeline(j)
    u2b = {v: k for k, v in byte_alphabet().items()}
    vocab = j["model"]["vocab"]
    n_vocab = max(vocab.values()) + 1
    tok = {}
    for s, i in vocab.items():
        try:
            tok[i] = bytes(u2b[ch] for ch in s)
        except KeyError:
            raise ValueError(f"vocab token {s!r} is not in the byte-level alphabet") from None
    byte_tok = np.full(256, -1, np.int32)
    for i, b in tok.items():
        if len(b) == 1:
            byte_tok[b[0]] = i
    if (byte_tok < 0).any():
        raise ValueError("the vocab lacks single-byte tokens")
    merges = {}
    for r, m in enumerate(j["model"]["merges"]):
        a, b = m.split(" ") if isinstance(m, str) else m
        ia, ib = vocab[a], vocab[b]
        merges[(ia, ib)] = (r, vocab[a + b])
    added = []
    for t in j.get("added_tokens", []):
        for f in ("single_word", "lstrip", "rstrip", "normalized"):
            if t.get(f):
                raise ValueError(f"added token {t['content']!r} has {f}")
        added.append((int(t["id"]), t["content"]))
    n_total = max([n_vocab] + [i + 1 for i, _ in added])
    dec = dict(tok)
    for i, content in added:   # HF ByteLevel decoder: alphabet chars map back to bytes, else UTF-8
        dec[i] = bytes(u2b[ch] for ch in content) if all(ch in u2b for ch in content) else content.encode("utf-8")
    ignore = bool(j["model"].get("ignore_merges"))
    direct = [i for i, b in tok.items() if len(b) > 1 and (ignore or _bpe([int(byte_tok[x]) for x in b], merges) == [i])]
    props, decomp, comp = tables if tables is not None else unicode_tables()

    sec: dict[int, bytes] = {}
    off = np.zeros(n_total + 1, np.uint32)
    blob = bytearray()
    for i in range(n_total):
        blob += dec.get(i, b"")
        off[i + 1] = len(blob)
    sec[20], sec[21], sec[22] = off.tobytes(), bytes(blob), byte_tok.tobytes()
    tbits = max(4, int(np.ceil(np.log2(max(1, len(direct)) * 2))) + 1)
    slots = np.zeros(1 << tbits, np.uint32)
    for i in direct:
        s = _hash_bytes(tok[i]) >> (64 - tbits)
        while slots[s]:
            s = (s + 1) & ((1 << tbits) - 1)
        slots[s] = i + 1
    sec[23] = slots.tobytes()
    mbits = max(4, int(np.ceil(np.log2(max(1, len(merges)) * 2))) + 1)
    mt = np.zeros(1 << mbits, np.dtype([("key", "<u8"), ("rank", "<u4"), ("id", "<u4")]))
    mt["key"] = np.uint64(0xFFFFFFFFFFFFFFFF)
    mask = (1 << mbits) - 1
    for (a, b), (r, i) in merges.items():
        key = (a << 32) | b
        s = ((key * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF) >> (64 - mbits)
        while mt["key"][s] != np.uint64(0xFFFFFFFFFFFFFFFF):
            s = (s + 1) & mask
        mt[s] = (key, r, i)
    sec[24] = mt.tobytes()
    atab, abytes = [], bytearray()
    for i, content in added:
        b = content.encode("utf-8")
        atab += [i, len(abytes), len(b)]
        abytes += b
    sec[25], sec[26] = np.array(atab, np.uint32).tobytes(), bytes(abytes)
    blocks, top = {}, np.zeros(NCP >> 8, np.uint16)
    for k in range(NCP >> 8):
        blk = props[k << 8:(k + 1) << 8].tobytes()
        top[k] = blocks.setdefault(blk, len(blocks))
    sec[27], sec[28] = top.tobytes(), b"".join(blocks)
    dk = sorted(decomp)
    dvals, ddata = [], []
    for c in dk:
        dvals.append((len(ddata) << 8) | len(decomp[c]))
        ddata += decomp[c]
    sec[29], sec[30], sec[31] = (np.array(dk, np.uint32).tobytes(), np.array(dvals, np.uint32).tobytes(),
                                 np.array(ddata, np.uint32).tobytes())
    ck = sorted(comp)
    sec[32] = np.array([(a << 21) | b for a, b in ck], np.uint64).tobytes()
    sec[33] = np.array([comp[k] for k in ck], np.uint32).tobytes()

    hdr = [0] * HDR_WORDS
    ids = {content: i for i, content in added}
    hdr[2:17] = [n_total, n_vocab, len(merges), len(added), max(len(b) for b in tok.values()), tbits, mbits,
                 ids.get("<|im_start|>", -1) & 0xFFFFFFFFFFFFFFFF, ids.get("<|im_end|>", -1) & 0xFFFFFFFFFFFFFFFF,
                 ids.get("<|endoftext|>", -1) & 0xFFFFFFFFFFFFFFFF, len(blocks), len(dk), len(ddata), len(ck), int(ignore)]
    body = bytearray()
    pos = HDR_WORDS * 8
    for k in range(20, 34):
        hdr[k] = pos + len(body)
        body += sec[k]
        body += b"\0" * (-len(body) % 8)
    hdr[0], hdr[1] = MAGIC, pos + len(body)
    Path(out).write_bytes(struct.pack(f"<{HDR_WORDS}Q", *hdr) + bytes(body))
    return {"n_total": n_total, "n_vocab": n_vocab, "merges": len(merges), "added": len(added),
            "direct": len(direct), "bytes": hdr[1]}


# ---- the native tokenizer ------------------------------------------------------------------

def _lib():
    from . import engine
    return engine.load_library()


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(_lib().ill_last_error().decode())


class Tokenizer:
    """Tokenizer(path:) over a compiled ILTK1 file (Tokenizer.swift:36-141), encoded and
    decoded by libillhip.so."""

    def __init__(self, path: str | os.PathLike):
        self._lib = _lib()
        h = C.c_void_p()
        _check(self._lib.ill_tok_open(os.fsencode(str(path)), C.byref(h)))
        self._h = h
        info = (C.c_int32 * 4)()
        _check(self._lib.ill_tok_info(self._h, info))
        self.vocab_size, self.im_start, self.im_end, self.end_of_text = (int(x) for x in info)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.ill_tok_close(self._h)
            self._h = None

    __del__ = close

    def _ids(self, call) -> list[int]:
        cap = 256
        while True:
            buf = (C.c_int32 * cap)()
            n = C.c_int64()
            rc = call(buf, cap, C.byref(n))
            if rc == 0:
                return buf[:n.value]
            if n.value <= cap:
                _check(rc)
            cap = n.value

    def encode(self, text: str) -> list[int]:
        """Plain text, no added-token matching (Tokenizer.encode, :150-152)."""
        b = text.encode("utf-8")
        return self._ids(lambda buf, cap, n: self._lib.ill_tok_encode(self._h, b, len(b), 0, buf, cap, n))

    def encode_with_specials(self, text: str) -> list[int]:
        """Added tokens matched leftmost-longest on the raw text (encodeWithSpecials, :154-158)."""
        b = text.encode("utf-8")
        return self._ids(lambda buf, cap, n: self._lib.ill_tok_encode(self._h, b, len(b), 1, buf, cap, n))

    def encode_chat(self, system: str, user: str) -> list[int]:
        """The chat template around (system, user) (encodeChat, :160-183)."""
        s, u = system.encode("utf-8"), user.encode("utf-8")
        return self._ids(lambda buf, cap, n: self._lib.ill_tok_encode_chat(self._h, s, len(s), u, len(u), buf, cap, n))

    def _bytes(self, call) -> bytes:
        cap = 1024
        while True:
            buf = C.create_string_buffer(cap)
            n = C.c_int64()
            rc = call(buf, cap, C.byref(n))
            if rc == 0:
                return buf.raw[:n.value]
            if n.value <= cap:
                _check(rc)
            cap = n.value

    def decode(self, ids) -> str:
        """Token bytes concatenated, invalid UTF-8 replaced by U+FFFD, unknown ids skipped
        (decode, :275-295)."""
        a = np.ascontiguousarray(np.asarray(list(ids), np.int32))
        p = a.ctypes.data_as(C.POINTER(C.c_int32))
        return self._bytes(lambda buf, cap, n: self._lib.ill_tok_decode(self._h, p, len(a), buf, cap, n)).decode("utf-8")

    def token_bytes(self, i: int) -> bytes:
        """Raw bytes of one id (tokenBytes, :266-271); empty for ids without a token."""
        p = C.c_char_p()
        n = C.c_int64()
        _check(self._lib.ill_tok_token_bytes(self._h, int(i), C.byref(p), C.byref(n)))
        return C.string_at(p, n.value) if n.value else b""

    def normalize(self, text: str) -> str:
        """The NFC normalization applied before pre-tokenization (normalize, :299-307)."""
        b = text.encode("utf-8")
        return self._bytes(lambda buf, cap, n: self._lib.ill_tok_normalize(self._h, b, len(b), buf, cap, n)).decode("utf-8")

    def pre_tokenize(self, text: str) -> list[bytes]:
        """Pre-tokenizer pieces of the normalized plain text, as raw bytes (preTokenize,
        :310-323)."""
        norm = self.normalize(text).encode("utf-8")
        cap = len(norm) + 1
        ends = (C.c_int64 * cap)()
        n = C.c_int64()
        _check(self._lib.ill_tok_pretokenize(self._h, norm, len(norm), ends, cap, C.byref(n)))
        out, a = [], 0
        for e in ends[:n.value]:
            out.append(norm[a:e])
            a = e
        return out

    @property
    def encode_fn(self):
        """(callback, user) for the C ABI's ill_encode_fn arguments (the learned drafter's
        request context): ill_tok_encode_cb with this tokenizer."""
        return self._lib.ill_tok_encode_cb, self._h


class TextStream:
    """Incremental detokenizer (TextStream, Tokenizer.swift:337-441): push ids as they are
    generated and get text that is safe to show; a trailing prefix of a well-formed UTF-8
    sequence is held back until a later token completes it. The chunks and finish() add up
    to decode(all ids)."""

    def __init__(self, tok: Tokenizer):
        self.tok = tok
        self.pending = b""

    @staticmethod
    def _proper_prefix(p: bytes, k: int) -> bool:
        c = p[k]
        lo, hi = {0xE0: (0xA0, 0xBF), 0xED: (0x80, 0x9F), 0xF0: (0x90, 0xBF), 0xF4: (0x80, 0x8F)}.get(c, (0x80, 0xBF))
        for i, d in enumerate(p[k + 1:]):
            if not (lo <= d <= hi if i == 0 else 0x80 <= d <= 0xBF):
                return False
        return True

    def push(self, i: int) -> str:
        b = self.tok.token_bytes(i)
        if not b:
            return ""
        self.pending += b
        p, n = self.pending, len(self.pending)
        keep = 0
        for k in range(n - 1, max(-1, n - 4), -1):
            c = p[k]
            if c & 0xC0 == 0x80:
                continue
            need = 2 if 0xC2 <= c <= 0xDF else 3 if 0xE0 <= c <= 0xEF else 4 if 0xF0 <= c <= 0xF4 else 1
            if need > n - k and self._proper_prefix(p, k):
                keep = n - k
            break
        out = p[:n - keep].decode("utf-8", errors="replace")
        self.pending = p[n - keep:]
        return out

    def finish(self) -> str:
        out = self.pending.decode("utf-8", errors="replace")
        self.pending = b""
        return out


def main(argv=None) -> int:
    import argparse
    ap = argparse.ArgumentParser(prog="python -m instantllm_amd.tokenizer")
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("compile", help="tokenizer.json -> ILTK1 file")
    c.add_argument("json")
    c.add_argument("out")
    e = sub.add_parser("encode", help="print the ids of a text")
    e.add_argument("file")
    e.add_argument("text")
    e.add_argument("--specials", action="store_true")
    d = sub.add_parser("decode", help="print the text of ids")
    d.add_argument("file")
    d.add_argument("ids", nargs="+", type=int)
    a = ap.parse_args(argv)
    if a.cmd == "compile":
        print(json.dumps(compile(a.json, a.out)))
    elif a.cmd == "encode":
        t = Tokenizer(a.file)
        print(" ".join(map(str, t.encode_with_specials(a.text) if a.specials else t.encode(a.text))))
    else:
        print(Tokenizer(a.file).decode(a.ids))
    return 0


if __name__ == "__main__":
    sys.exit(main())
