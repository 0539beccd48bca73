"""The native tokenizer (instantllm_amd/tokenizer.py + csrc/ill_tok.h) against Hugging Face
`tokenizers`, the library the reference's tokenizer is defined by and checked against
(its goldens come from `tokenizers`: /root/reference/tools/tokenizer_golden.py:1-26; its
Unicode tables are probed from it: tools/tokenizer_unicode.py:1-20).

No Qwen tokenizer.json ships in this image, so the tests train a byte-level BPE with the
Qwen2 pipeline (NFC, the Qwen2 split regex, byte-level BPE and decoder, Qwen2.5's added
tokens) with `tokenizers` itself, compile it, and compare every encoding mode, the NFC
normalization, the pre-tokenizer, decoding and streaming with what `tokenizers` returns on
the same tokenizer.json: hand-written edge cases of the categories the reference's goldens
cover (contractions and their case folds, whitespace runs, CR/LF, digits, punctuation,
code, paths, CJK, emoji sequences, NFC-sensitive text, Hangul jamo, RTL scripts, control
characters, added tokens and fragments of them), random strings over a hard alphabet, every
code point in context, long pieces, random id sequences, and two hand-made vocabularies for
the rules a trained one never exercises (a token its own bytes do not merge into, and
`ignore_merges`). Host code only: no GPU."""
from __future__ import annotations

import ctypes as C
import json
import random
import sysconfig
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "instantllm_amd" / "libillhip.so"
pytestmark = pytest.mark.skipif(not LIB.exists(), reason="libillhip.so not built (run __graft_entry__.build())")
tokenizers = pytest.importorskip("tokenizers")

from instantllm_amd import tokenizer as TK  # noqa: E402

QWEN_ADDED = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|object_ref_start|>", "<|object_ref_end|>",
              "<|box_start|>", "<|box_end|>", "<|quad_start|>", "<|quad_end|>", "<|vision_start|>", "<|vision_end|>",
              "<|vision_pad|>", "<|image_pad|>", "<|video_pad|>", "<tool_call>", "</tool_call>", "<|fim_prefix|>",
              "<|fim_middle|>", "<|fim_suffix|>", "<|fim_pad|>", "<|repo_name|>", "<|file_sep|>"]

EDGE = [
    "", " ", "   ", "\n", "\r\n", "\r", "\t", "\v", "\f", "x", "7", "'", "''", "'''",
    # contractions: every letter, both cases, the long s and Kelvin sign, near misses
    "'s", "'S", "'\u017f", "'t", "'T", "'re", "'RE", "'rE", "'ve", "'Ve", "'m", "'M", "'ll", "'LL", "'lL", "'d", "'D",
    "'q", "'r", "'l", "'lq", "'rent", "'verb", "'done", "'Sam", "'mine", "'til", "'\u212a", "'\u0130", "'\u017fe",
    "we've", "WE'VE", "you'd", "it'll", "IT'LL", "they're", "she's", "I'M", "won't", "Won'T", "o'clock",
    "'s's's", " 's", "\t's", "\n's", "z's", "9's", "?'s", "''s", "'4", "' s", "don\u2019t", "\u2018hi\u2019",
    "He said 'Sure, I'D go' and 'LL see; we'Re 'vE 'M", "'re'", "''ll", "'ll've", "rock'n'roll",
    # numbers in several scripts
    "0", "42", "31415", "2.718", "-7", "+6e-3", "10,000", "0xFF", "v3.10.12", "99%", "$4.50", "\u00b2", "\u00be",
    "\u2167", "\u0664\u0665", "\u096a\u096b", "\u2463", "\U0001d7ce", "\uff17\uff18", "x86_64", "2026-12-02 13:45",
    "10.0.0.1", "1e-9", "7/8", "#42", "r2d2c3po",
    # whitespace of every kind
    "p  q", "p   q", "p \n q", "p\n\nq", "p\r\n\r\nq", "p\t\tq", "\t\tp", "  \n  p", " \n", "\n ", "p \n ",
    "\u00a0p", "p\u00a0\u00a0q", "\u3000p", "p\u3000\u3000q", "p\u2028q", "p\u2029q", "p\u0085q", "p\u000bq",
    "\u200bp", "\ufeffp", "pq   ", "   pq", " \t \n \t ", "\n\n\n", "\r\r\n", "p\rq", "\n\r", "p \u00a0q",
    "\u1680p", "\u2002\u2003p", "\u202fp", "\u205fp", "p\x1cq\x1dr\x1e\x1f", "p \t3", "p  3", " 3", "\t3", "\n3",
    " ?", "  ?", "\t?", "\n?", "one  \n  two", "one \r\n two", "l1\r\nl2\r\n", "end \n", "  \n\n  \n",
    # punctuation and code
    "???", "..", "p..q", "(a)", "[b]", "{c}", "f()", "i-=2", "p->q", "p=>q", "p::q", "p//q", "#!/usr/bin/env sh",
    "<<END", "&&", "||", "@property", "$PATH", "${X}", "%d", "\\t", "\"s\"", "`ls`", "??\n\n", " ?\n", ".\r\n",
    "if x:\n    return 1\n", "while (i < n) {\n\ti++;\n}\r\n", "SELECT a FROM t;", "<p id=\"q\">r</p>", "<>",
    # shell, paths, URLs
    "ls -lh /tmp | sort -k5", "grep -rn 'TODO' src/", "ssh user@host -p 2222", "/opt/rocm/bin/hipcc",
    "C:\\Program Files\\x.exe", "~/.config/app/", "https://host.example/p?a=1&b=2#top", "mailto:a@b.c",
    # CJK, emoji sequences
    "\u6e2c\u8a66\u6587\u5b57", "\u3072\u3089\u304c\u306a\u30ab\u30bf\u30ab\u30ca", "\uc870\uc120\uae00 \ud55c\uae00",
    "\u6f22\u5b57mixed\u6587\u5b57", "\U0001f642", "\U0001f44b\U0001f3fe", "\U0001f468\u200d\U0001f469\u200d\U0001f466",
    "\U0001f3f4\u200d\u2620\ufe0f", "\U0001f1e9\U0001f1ea", "2\ufe0f\u20e3", "\u2764\ufe0f\u200d\U0001f525",
    " \U0001f642", "\U0001f642\U0001f642", "\U0001f642ok", "ok\U0001f642",
    # NFC: composed and decomposed, reordering, blocking, singletons, exclusions, Hangul
    "na\u00efve", "nai\u0308ve", "o\u0302\u0301", "a\u0328\u0301", "a\u0301\u0328", "\u1100\u1162\u11ab",
    "\u1101\u1161", "\uac01\u11a8", "\u212b", "\u2126", "\u0929", "\u095c", "\ufb00", "\u01db", "\u1e9b\u0323",
    "s\u0323\u0307", "s\u0307\u0323", "\u0344", "\u0f75", "\u00d6\u0304", "\u017f\u0307", "u\u0308\u0300",
    "\u0301start", " \u0301", "\u0301\u0301", "p\u0301\u0327q", "Vi\u00ea\u0323t Nam", "\u00e8" * 40, "e\u0300" * 40,
    "\u0928\u093c", "\u09c7\u09d7", "\u0b47\u0b56", "\u0bc6\u0bd7", "\u0cc6\u0cc2", "\u0d46\u0d57", "\u0dd9\u0ddf",
    "\u0627\u0654", "\u05d0\u05b7\u05bc", "\u05d0\u05bc\u05b7",
    # other scripts, RTL
    "\u0627\u0644\u0633\u0644\u0627\u0645", "\u05d1\u05e8\u05d5\u05da", "\u0639\u0631\u0628\u064a 7 Latin",
    "\u202eabc\u202c", "\u0939\u093f\u0928\u094d\u0926\u0940", "\u0e20\u0e32\u0e29\u0e32\u0e44\u0e17\u0e22",
    "\u0395\u03bb\u03bb\u03b7\u03bd\u03b9\u03ba\u03ac", "\u0420\u0443\u0441\u0441\u043a\u0438\u0439", "\u10e5\u10d0\u10e0\u10d7\u10e3\u10da\u10d8",
    "\u0540\u0561\u0575", "\u12a0\u121b\u122d\u129b", "\u0ba4\u0bae\u0bbf\u0bb4\u0bcd", "\u1781\u17d2\u1798\u17c2\u179a",
    # symbols, fullwidth, control characters
    "\u2203y\u2209S", "\u2264\u2265\u2260", "\u221b8", "\uff28\uff49\uff01", "\uff8a\uff9d\uff76\uff78", "\u00ae\u2122",
    "\u2014\u2013", "\u00bb\u00ab", "\u2026", "\x00", "p\x00q", "\x1b[1mB\x1b[0m", "\x7f", "\x02\x03", "\x08",
    # added tokens and fragments of them
    "<|im_start|>", "<|im_end|>", "<|endoftext|>", "<|im_start|>user\nyo<|im_end|>", "<|im_start", "im_end|>",
    "<|im_start|><|im_end|>", "<<|im_end|>>", "<|IM_END|>", "p<|endoftext|>q", " <|im_end|> ", "<|im",
    "<|im<|im_end|>", "<tool_call>{\"f\": 1}</tool_call>", "<|fim_prefix|>a<|fim_suffix|>b<|fim_middle|>",
    "<|vision_start|><|image_pad|><|vision_end|>", "<|file_sep|>x.py\n", "<|endoftext|>" * 3, "<" * 4, "<|",
    "|>", "e<|im_end|>\u0301", "\u0301<|im_start|>", "<tool_call", "x</tool_call>y", "  <|endoftext|>  ",
]
SYSTEM = "You are a terse assistant. Answer with one line."
PROMPTS = ["list the files in this folder", "what is 17 * 23?", "summarize: the quick brown fox",
           "\u00bfd\u00f3nde est\u00e1 la estaci\u00f3n?", "\u7ffb\u8bd1\u8fd9\u53e5\u8bdd", "fix 'it's' vs 'its'"]
HARD = list("aAsStTmMdDrReEvVlLqQ'\u2019 \t\n\r.,;!?-_#<>|0123456789") + \
    [" ", "\u3000", "\u00a0", "\u00e9", "e\u0301", "\u0308", "\u0323", "\u017f", "\u00df", "\u4e2d", "\ud55c", "\u1100",
     "\u1161", "\u11a8", "\U0001f642", "\u200d", "<|im_end|>", "<|im_start|>", "<|im", "<tool_call>", "\u0664"]


def _corpus():
    lib = Path(sysconfig.get_paths()["stdlib"])
    for f in sorted(lib.glob("*.py"))[:80]:
        yield f.read_text(encoding="utf-8", errors="replace")
    yield "\n".join(EDGE + PROMPTS)


def _train(out: Path) -> Path:
    from tokenizers import AddedToken, Regex, Tokenizer, decoders, models, normalizers, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE())
    tok.normalizer = normalizers.NFC()
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(TK.QWEN2_SPLIT), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    tok.train_from_iterator(_corpus(), trainers.BpeTrainer(vocab_size=6000, show_progress=False,
                                                           initial_alphabet=pre_tokenizers.ByteLevel.alphabet()))
    tok.add_tokens([AddedToken(s, special=True, normalized=False) for s in QWEN_ADDED[:3]])
    tok.add_tokens([AddedToken(s, special=False, normalized=False) for s in QWEN_ADDED[3:] + ["<|im"]])
    p = out / "tokenizer.json"
    tok.save(str(p))
    return p


@pytest.fixture(scope="module")
def env(tmp_path_factory):
    from tokenizers import Tokenizer
    d = tmp_path_factory.mktemp("tok")
    tables = TK.unicode_tables()
    src = _train(d)
    TK.compile(src, d / "t.iltk", tables=tables)
    j = json.loads(src.read_text(encoding="utf-8"))
    j["added_tokens"] = []
    return {"hf": Tokenizer.from_file(str(src)), "plain": Tokenizer.from_str(json.dumps(j)), "me": TK.Tokenizer(d / "t.iltk"),
            "dir": d, "tables": tables, "json": src}


def _mismatches(env, texts):
    from tokenizers import normalizers
    nfc = normalizers.NFC()
    hf, plain, me = env["hf"], env["plain"], env["me"]
    bad = []
    for s in texts:
        got = (me.encode(s), me.encode_with_specials(s), me.normalize(s))
        want = (plain.encode(s, add_special_tokens=False).ids, hf.encode(s, add_special_tokens=False).ids, nfc.normalize_str(s))
        if got != want:
            bad.append(s)
    return bad


def test_edge_cases(env):
    texts = EDGE + ["".join(EDGE), "\n".join(EDGE), " ".join(EDGE)] + PROMPTS
    assert _mismatches(env, texts) == []


def test_random_strings(env):
    rng = random.Random(11)
    texts = ["".join(rng.choice(HARD) for _ in range(rng.randint(1, 24))) for _ in range(4000)]
    assert _mismatches(env, texts) == []


def test_every_code_point_in_context(env):
    """Each code point between letters, and doubled after an apostrophe and a space: the
    split classes, the contraction folds and NFC of every code point as `tokenizers` has them."""
    cps = [c for c in range(0x110000) if not 0xD800 <= c <= 0xDFFF]
    texts = []
    for k in range(0, len(cps), 4096):
        chunk = cps[k:k + 4096]
        texts.append("".join("a%sb|" % chr(c) for c in chunk))
        texts.append("".join("'%s%s |" % (chr(c), chr(c)) for c in chunk))
    assert _mismatches(env, texts) == []


def test_nfc_sequences(env):
    """Random runs of combining marks (reordering, blocked and unblocked compositions),
    decomposable characters and Hangul jamo, against the NFC of `tokenizers`."""
    from tokenizers import normalizers
    props, decomp, comp = env["tables"]
    nfc = normalizers.NFC()
    marks = [c for c in range(0x300, 0x370)] + [0x323, 0x328, 0x31b, 0x5b7, 0x5bc, 0x93c, 0x3099, 0x309a]
    starters = sorted({a for a, _ in comp})[:400] + list(range(0x1100, 0x1113)) + list(range(0xAC00, 0xAC40))
    seconds = sorted({b for _, b in comp}) + list(range(0x1161, 0x1176)) + list(range(0x11A8, 0x11C3))
    pool = marks + starters + seconds + sorted(decomp)[:2000] + [ord(x) for x in "abc "]
    rng = random.Random(5)
    texts = ["".join(chr(rng.choice(pool)) for _ in range(rng.randint(1, 12))) for _ in range(6000)]
    me = env["me"]
    assert [s for s in texts if me.normalize(s) != nfc.normalize_str(s)] == []
    # the fast path's premise: a text of code points without the flag is NFC already, and
    # no flagged code point lies below U+0300 (their UTF-8 lead bytes are skipped)
    plain = [c for c in range(0x300, 0x3000) if not props[c] & TK.F_NFC]
    texts = ["".join(chr(rng.choice(plain)) for _ in range(rng.randint(1, 12))) for _ in range(3000)]
    assert [s for s in texts if nfc.normalize_str(s) != s] == []
    assert not any(props[c] & TK.F_NFC for c in range(0x300))


def test_long_pieces(env):
    """Pieces past 64 bytes take the heap merge path."""
    rng = random.Random(3)
    texts = ["q" * 500, "ab" * 300, "abc" * 200, " " * 700, "\n" * 200, "=" * 300, "-=" * 200, "\U0001f642" * 60,
             "\u6587" * 400, "".join(rng.choice("etaoinshrdlu") for _ in range(3000)),
             "".join(rng.choice("ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz") for _ in range(2000)),
             "a\u0301" * 200, "\u00e0" * 200, "x" * 63, "x" * 64, "x" * 65, " " * 64 + "y", "'s" * 100]
    assert _mismatches(env, texts) == []


def test_chat_template(env):
    hf, me = env["hf"], env["me"]
    for s in [SYSTEM, "", " ", "<|im_end|>"] + EDGE[::7]:
        for u in PROMPTS[:3] + ["", "\n", "<|im_start|>x"]:
            want = hf.encode(TK.CHAT_TEMPLATE.format(s=s, u=u), add_special_tokens=False).ids
            assert me.encode_chat(s, u) == want, (s, u)


def test_pretokenize(env):
    """The pieces of the split regex, as `tokenizers`' Split pre-tokenizer cuts them."""
    from tokenizers import Regex, normalizers, pre_tokenizers
    sp = pre_tokenizers.Split(Regex(TK.QWEN2_SPLIT), behavior="isolated")
    nfc = normalizers.NFC()
    rng = random.Random(8)
    texts = EDGE + ["".join(rng.choice(HARD) for _ in range(rng.randint(1, 30))) for _ in range(1500)]
    me = env["me"]
    for s in texts:
        want = [p.encode("utf-8") for p, _ in sp.pre_tokenize_str(nfc.normalize_str(s))]
        assert me.pre_tokenize(s) == want, s


def test_decode_and_stream(env):
    hf, me = env["hf"], env["me"]
    n = me.vocab_size
    rng = random.Random(9)
    for _ in range(3000):
        ids = [rng.randrange(-2, n + 3) for _ in range(rng.randint(0, 24))]
        want = hf.decode([i for i in ids if 0 <= i < n], skip_special_tokens=False)
        assert me.decode(ids) == want, ids
        st = TK.TextStream(me)
        got = "".join(st.push(i) for i in ids) + st.finish()
        assert got == want, ids
    for s in EDGE:
        ids = me.encode_with_specials(s)
        assert me.decode(ids) == hf.decode(ids, skip_special_tokens=False)


def test_info_and_callback(env):
    me = env["me"]
    hf = env["hf"]
    assert me.vocab_size == hf.get_vocab_size(with_added_tokens=True)
    assert (me.im_start, me.im_end, me.end_of_text) == tuple(hf.token_to_id(t) for t in ("<|im_start|>", "<|im_end|>", "<|endoftext|>"))
    fn, h = me.encode_fn
    buf = (C.c_int32 * 8)()
    text = "hello <|im_end|> world, it's 3 o'clock"
    want = me.encode_with_specials(text)
    assert len(want) > 8
    assert fn(h, text.encode(), buf, 8) == len(want)
    assert list(buf) == want[:8]


def test_drafter_context_with_native_tokenizer(env, tmp_path):
    """The learned drafter's request context (ill_ildraft_prepare) takes the library's own
    tokenizer callback: the same context as with a Python function over the same tokenizer."""
    import sys
    sys.path.insert(0, str(ROOT / "tests" / "golden"))
    from make_ildraft_fixtures import make_table
    from instantllm_amd.engine import DraftTable
    blob, reqs = make_table()
    p = tmp_path / "t.bin"
    p.write_bytes(blob)
    me = env["me"]
    d = DraftTable(str(p))
    try:
        for r in reqs:
            a = d.prepare(r["pids"], r["prompt"], me)
            b = d.prepare(r["pids"], r["prompt"], me.encode_with_specials)
            assert a.tobytes() == b.tobytes()
    finally:
        d.close()


def test_errors(env):
    me = env["me"]
    lib = me._lib
    n = C.c_int64()
    buf = (C.c_int32 * 16)()
    for bad in (b"\xff", b"a\xc3", b"\xed\xa0\x80", b"\xf4\x90\x80\x80", b"\xc0\xaf"):
        assert lib.ill_tok_encode(me._h, bad, len(bad), 0, buf, 16, C.byref(n)) == TK_E_ARG
    # a buffer too small reports the count it needs
    need = len(me.encode("a b c d e"))
    assert need > 2
    assert lib.ill_tok_encode(me._h, b"a b c d e", 9, 0, buf, 2, C.byref(n)) == TK_E_ARG and n.value == need
    h = C.c_void_p()
    d = env["dir"]
    (d / "junk.iltk").write_bytes(b"\0" * 4096)
    assert lib.ill_tok_open(str(d / "junk.iltk").encode(), C.byref(h)) == TK_E_FILE
    assert lib.ill_tok_open(str(d / "missing.iltk").encode(), C.byref(h)) == TK_E_FILE
    raw = (d / "t.iltk").read_bytes()
    (d / "short.iltk").write_bytes(raw[:len(raw) // 2])
    assert lib.ill_tok_open(str(d / "short.iltk").encode(), C.byref(h)) == TK_E_FILE
    j = json.loads(env["json"].read_text(encoding="utf-8"))
    for edit in (lambda j: j.update(normalizer=None),
                 lambda j: j["pre_tokenizer"]["pretokenizers"][0]["pattern"].update(Regex="\\s+"),
                 lambda j: j["added_tokens"][0].update(normalized=True)):
        k = json.loads(json.dumps(j))
        edit(k)
        (d / "bad.json").write_text(json.dumps(k), encoding="utf-8")
        with pytest.raises(ValueError):
            TK.compile(d / "bad.json", d / "bad.iltk", tables=env["tables"])


TK_E_ARG, TK_E_FILE = -1, -2


def _handmade(ignore: bool) -> dict:
    """Byte-level alphabet plus 'ab', 'bc', 'abc' with merges (b c) < (a b) < (ab c): merging
    the bytes of 'abc' gives a + bc, so 'abc' is a token its own bytes never reach."""
    alpha = TK.byte_alphabet()
    vocab = {alpha[b]: b for b in range(256)}
    for s in ("ab", "bc", "abc"):
        vocab[s] = len(vocab)
    j = {"version": "1.0", "truncation": None, "padding": None, "added_tokens": [
        {"id": len(vocab), "content": "<|im_start|>", "single_word": False, "lstrip": False, "rstrip": False,
         "normalized": False, "special": True},
        {"id": len(vocab) + 1, "content": "<|im_end|>", "single_word": False, "lstrip": False, "rstrip": False,
         "normalized": False, "special": True}],
         "normalizer": {"type": "NFC"},
         "pre_tokenizer": {"type": "Sequence", "pretokenizers": [
             {"type": "Split", "pattern": {"Regex": TK.QWEN2_SPLIT}, "behavior": "Isolated", "invert": False},
             {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False}]},
         "post_processor": None,
         "decoder": {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False},
         "model": {"type": "BPE", "dropout": None, "unk_token": None, "continuing_subword_prefix": "", "end_of_word_suffix": "",
                   "fuse_unk": False, "byte_fallback": False, "ignore_merges": ignore, "vocab": vocab,
                   "merges": [["b", "c"], ["a", "b"], ["ab", "c"]]}}
    return j


@pytest.mark.parametrize("ignore", [False, True])
def test_unreachable_token_and_ignore_merges(env, ignore):
    from tokenizers import Tokenizer
    d = env["dir"]
    j = _handmade(ignore)
    p = d / f"hand{int(ignore)}.json"
    p.write_text(json.dumps(j), encoding="utf-8")
    hf = Tokenizer.from_file(str(p))
    TK.compile(p, d / f"hand{int(ignore)}.iltk", tables=env["tables"])
    me = TK.Tokenizer(d / f"hand{int(ignore)}.iltk")
    for s in ("abc", "abcabc", " abc", "ab", "bc", "xabc", "abcd", "c abc b<|im_end|>abc", "a" * 80 + "bc" * 40):
        assert me.encode_with_specials(s) == hf.encode(s, add_special_tokens=False).ids, s
    want_abc = [j["model"]["vocab"]["abc"]] if ignore else [j["model"]["vocab"]["a"], j["model"]["vocab"]["bc"]]
    assert me.encode("abc") == want_abc
