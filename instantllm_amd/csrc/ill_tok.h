// Qwen2 byte-level BPE tokenizer over a compiled ILTK1 file (written by
// instantllm_amd/tokenizer.py from a Hugging Face tokenizer.json): the reference's
// Sources/Tokenizer (Tokenizer.swift, Core.swift) on the Linux host. Host code only.
//
// Encoding follows Hugging Face `tokenizers` for the Qwen2 pipeline:
//   1. (with added tokens) the text is cut at added tokens, leftmost first and longest at a
//      position, matched on the raw bytes (Tokenizer.swift:242-280);
//   2. every other segment is NFC-normalized (canonical decomposition, canonical ordering,
//      canonical composition, Hangul algorithmically; Core.swift:437-524), skipped when no
//      code point in it may change;
//   3. the segment is cut into pieces by the Qwen2 split regex
//        (?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*
//        |\s*[\r\n]+|\s+(?!\S)|\s+
//      with Oniguruma's leftmost-first alternation, written out below as a function of the
//      character classes of the piece's first characters (Core.swift:113-210);
//   4. a one-byte piece is its byte's token; a piece whose bytes are a token that byte-pair
//      merging of those bytes reaches (the compiler's direct table) is that token; any other
//      piece is merged pair by pair, the lowest merge rank first and the leftmost of equal
//      ranks, which is the order of HF's (rank, position) heap (Core.swift:229-380).
// Decoding concatenates the tokens' bytes (added tokens through the byte-level decoder, as
// the compiler stored them) and replaces ill-formed UTF-8 by U+FFFD per maximal subpart, as
// Rust's from_utf8_lossy does.
#pragma once
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace iltk {

constexpr uint64_t kMagic = 0x31304B544C49ull;   // "ILTK01"
constexpr int kHdrWords = 64;
enum Cls { kL = 0, kN = 1, kO = 2, kWS = 3, kSP = 4, kNL = 5 };
constexpr uint16_t kNFC = 1 << 3, kC1 = 1 << 4, kRV = 1 << 5, kE = 1 << 6, kLL = 1 << 7;
constexpr uint32_t kSBase = 0xAC00, kLBase = 0x1100, kVBase = 0x1161, kTBase = 0x11A7;
constexpr uint32_t kLCount = 19, kVCount = 21, kTCount = 28, kNCount = 21 * 28, kSCount = 19 * 21 * 28;

struct MergeSlot {
  uint64_t key;
  uint32_t rank, id;
};

struct Tok {
  void* map = nullptr;
  size_t size = 0;
  int64_t n_total = 0, n_vocab = 0, n_added = 0, max_len = 0;
  int tbits = 0, mbits = 0;
  int32_t im_start = -1, im_end = -1, eot = -1;
  const uint32_t* tok_off = nullptr;
  const uint8_t* tok_bytes = nullptr;
  const int32_t* byte_tok = nullptr;
  const uint32_t* tok_slots = nullptr;
  const MergeSlot* merges = nullptr;
  const uint32_t* added = nullptr;
  const uint8_t* added_bytes = nullptr;
  const uint16_t* uni_top = nullptr;
  const uint16_t* uni_blocks = nullptr;
  const uint32_t* dkeys = nullptr;
  const uint32_t* dvals = nullptr;
  const uint32_t* ddata = nullptr;
  const uint64_t* ckeys = nullptr;
  const uint32_t* cvals = nullptr;
  int64_t n_dec = 0, n_ddata = 0, n_comp = 0, n_blocks = 0;
  bool first_byte[256] = {};   // bytes an added token starts with
  std::string chat0, chat1, chat2;   // the chat template around {system} and {user}

  ~Tok() {
    if (map) munmap(map, size);
  }

  // ---- Unicode ----
  uint16_t prop(uint32_t cp) const { return cp < 0x110000 ? uni_blocks[(size_t)uni_top[cp >> 8] * 256 + (cp & 255)] : (uint16_t)kO; }
  int ccc(uint32_t cp) const { return prop(cp) >> 8; }
};

// Hash of a token's bytes (FNV-1a 64, the compiler's _hash_bytes).
inline uint64_t hash_bytes(const uint8_t* p, size_t n) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (size_t i = 0; i < n; i++) h = (h ^ p[i]) * 0x100000001B3ull;
  return h;
}

// Length of the well-formed UTF-8 sequence at p[i] (0: ill-formed), and its code point.
inline int utf8_at(const uint8_t* p, size_t i, size_t n, uint32_t* cp) {
  const uint8_t b = p[i];
  if (b < 0x80) {
    *cp = b;
    return 1;
  }
  int len;
  uint8_t lo = 0x80, hi = 0xBF;
  if (b >= 0xC2 && b <= 0xDF) len = 2;
  else if (b >= 0xE0 && b <= 0xEF) {
    len = 3;
    if (b == 0xE0) lo = 0xA0;
    if (b == 0xED) hi = 0x9F;
  } else if (b >= 0xF0 && b <= 0xF4) {
    len = 4;
    if (b == 0xF0) lo = 0x90;
    if (b == 0xF4) hi = 0x8F;
  } else {
    return 0;
  }
  if (i + len > n) return 0;
  if (p[i + 1] < lo || p[i + 1] > hi) return 0;
  uint32_t c = b & (0x7F >> len);
  for (int k = 1; k < len; k++) {
    if (k > 1 && (p[i + k] & 0xC0) != 0x80) return 0;
    c = (c << 6) | (p[i + k] & 0x3F);
  }
  *cp = c;
  return len;
}

inline bool utf8_valid(const uint8_t* p, size_t n) {
  uint32_t cp;
  for (size_t i = 0; i < n;) {
    const int l = utf8_at(p, i, n, &cp);
    if (!l) return false;
    i += l;
  }
  return true;
}

inline void put_utf8(uint32_t c, std::string& out) {
  if (c < 0x80) {
    out += (char)c;
  } else if (c < 0x800) {
    out += (char)(0xC0 | (c >> 6));
    out += (char)(0x80 | (c & 0x3F));
  } else if (c < 0x10000) {
    out += (char)(0xE0 | (c >> 12));
    out += (char)(0x80 | ((c >> 6) & 0x3F));
    out += (char)(0x80 | (c & 0x3F));
  } else {
    out += (char)(0xF0 | (c >> 18));
    out += (char)(0x80 | ((c >> 12) & 0x3F));
    out += (char)(0x80 | ((c >> 6) & 0x3F));
    out += (char)(0x80 | (c & 0x3F));
  }
}

// Bytes as UTF-8 with each maximal ill-formed subpart replaced by U+FFFD.
inline std::string lossy_utf8(const uint8_t* p, size_t n) {
  std::string out;
  out.reserve(n);
  uint32_t cp;
  for (size_t i = 0; i < n;) {
    const int l = utf8_at(p, i, n, &cp);
    if (l) {
      out.append((const char*)p + i, l);
      i += l;
      continue;
    }
    // the maximal subpart: a lead byte and the continuation bytes that still fit it
    const uint8_t b = p[i];
    size_t k = 1;
    int len = b >= 0xC2 && b <= 0xDF ? 2 : b >= 0xE0 && b <= 0xEF ? 3 : b >= 0xF0 && b <= 0xF4 ? 4 : 1;
    if (len > 1 && i + 1 < n) {
      const uint8_t lo = b == 0xE0 ? 0xA0 : b == 0xF0 ? 0x90 : 0x80, hi = b == 0xED ? 0x9F : b == 0xF4 ? 0x8F : 0xBF;
      if (p[i + 1] >= lo && p[i + 1] <= hi) {
        k = 2;
        while ((int)k < len && i + k < n && (p[i + k] & 0xC0) == 0x80) k++;
      }
    }
    out += "\xEF\xBF\xBD";
    i += k;
  }
  return out;
}

// ---- NFC -----------------------------------------------------------------------------
inline bool needs_nfc(const Tok& t, const uint8_t* p, size_t n) {
  uint32_t cp;
  for (size_t i = 0; i < n;) {
    if (p[i] < 0xCC) {   // code points below U+0300 never change under NFC
      i++;
      continue;
    }
    const int l = utf8_at(p, i, n, &cp);
    if (t.prop(cp) & kNFC) return true;
    i += l;
  }
  return false;
}

inline void decompose(const Tok& t, uint32_t c, std::vector<uint32_t>& out) {
  if (c >= kSBase && c < kSBase + kSCount) {
    const uint32_t s = c - kSBase;
    out.push_back(kLBase + s / kNCount);
    out.push_back(kVBase + (s % kNCount) / kTCount);
    if (s % kTCount) out.push_back(kTBase + s % kTCount);
    return;
  }
  const uint32_t* e = t.dkeys + t.n_dec;
  const uint32_t* f = std::lower_bound(t.dkeys, e, c);
  if (f != e && *f == c) {
    const uint32_t v = t.dvals[f - t.dkeys];
    out.insert(out.end(), t.ddata + (v >> 8), t.ddata + (v >> 8) + (v & 255));
    return;
  }
  out.push_back(c);
}

// The primary composite of (a, b), or 0.
inline uint32_t compose(const Tok& t, uint32_t a, uint32_t b) {
  if (a >= kLBase && a < kLBase + kLCount && b >= kVBase && b < kVBase + kVCount)
    return kSBase + ((a - kLBase) * kVCount + (b - kVBase)) * kTCount;
  if (a >= kSBase && a < kSBase + kSCount && (a - kSBase) % kTCount == 0 && b > kTBase && b < kTBase + kTCount)
    return a + (b - kTBase);
  const uint64_t key = ((uint64_t)a << 21) | b;
  const uint64_t* e = t.ckeys + t.n_comp;
  const uint64_t* f = std::lower_bound(t.ckeys, e, key);
  return f != e && *f == key ? t.cvals[f - t.ckeys] : 0u;
}

inline void nfc(const Tok& t, const uint8_t* p, size_t n, std::string& out) {
  std::vector<uint32_t> cps;
  cps.reserve(n + 8);
  uint32_t cp;
  for (size_t i = 0; i < n;) {
    i += utf8_at(p, i, n, &cp);
    decompose(t, cp, cps);
  }
  // canonical ordering: each run of non-starters sorted stably by class
  const size_t m = cps.size();
  for (size_t a = 0; a < m;) {
    if (!t.ccc(cps[a])) {
      a++;
      continue;
    }
    size_t e = a;
    while (e < m && t.ccc(cps[e])) e++;
    std::stable_sort(cps.begin() + a, cps.begin() + e, [&](uint32_t x, uint32_t y) { return t.ccc(x) < t.ccc(y); });
    a = e;
  }
  // canonical composition: a character joins the last starter unless a character between
  // them has class 0 or a class >= its own
  size_t w = 0;
  long starter = -1;
  int last = -1;   // class of the last character kept after the starter (-1: none)
  for (size_t x = 0; x < m; x++) {
    const uint32_t c = cps[x];
    const int k = t.ccc(c);
    if (starter >= 0 && (last == -1 || last < k)) {
      const uint32_t r = compose(t, cps[starter], c);
      if (r) {
        cps[starter] = r;
        continue;
      }
    }
    if (k == 0) {
      starter = (long)w;
      last = -1;
    } else if (starter >= 0) {
      last = k;
    }
    cps[w++] = c;
  }
  for (size_t x = 0; x < w; x++) put_utf8(cps[x], out);
}

// ---- pre-tokenizer -------------------------------------------------------------------
// Class and flags of the character at p[i] (valid UTF-8), and its length.
inline uint16_t prop_at(const Tok& t, const uint8_t* p, size_t i, size_t n, int* len) {
  uint32_t cp;
  *len = utf8_at(p, i, n, &cp);
  return t.prop(cp);
}

// End of the run of characters of class `cls` from j.
inline size_t run_of(const Tok& t, const uint8_t* p, size_t j, size_t n, int cls) {
  int l;
  while (j < n && (prop_at(t, p, j, n, &l) & 7) == cls) j += l;
  return j;
}

inline size_t nl_run(const uint8_t* p, size_t j, size_t n) {
  while (j < n && (p[j] == '\r' || p[j] == '\n')) j++;
  return j;
}

// Whitespace starting at i: \s*[\r\n]+ (to the run's last CR / LF), else \s+(?!\S) (the run
// to the end, or the run without its last character), else \s+ (one character).
inline size_t ws_piece(const Tok& t, const uint8_t* p, size_t i, size_t n) {
  size_t j = i, last_nl = (size_t)-1, last_start = i;
  int l;
  while (j < n) {
    const int c = prop_at(t, p, j, n, &l) & 7;
    if (c < kWS) break;
    if (c == kNL) last_nl = j;
    last_start = j;
    j += l;
  }
  if (last_nl != (size_t)-1) return last_nl + 1;
  if (j == n) return n;
  if (last_start > i) return last_start;
  return j;
}

// (?i:'s|'t|'re|'ve|'m|'ll|'d) after an apostrophe ending at k: the contraction's end or 0.
inline size_t contraction(const Tok& t, const uint8_t* p, size_t k, size_t n) {
  if (k >= n) return 0;
  int l1, l2;
  const uint16_t a = prop_at(t, p, k, n, &l1);
  if (a & kC1) return k + l1;
  if ((a & (kRV | kLL)) && k + l1 < n) {
    const uint16_t b = prop_at(t, p, k + l1, n, &l2);
    if (((a & kRV) && (b & kE)) || ((a & kLL) && (b & kLL))) return k + l1 + l2;
  }
  return 0;
}

// End of the piece starting at i: the first alternative of the split regex that matches.
inline size_t piece_end(const Tok& t, const uint8_t* p, size_t i, size_t n) {
  int l, l2;
  const int c = prop_at(t, p, i, n, &l) & 7;
  const size_t j = i + l;
  switch (c) {
    case kL:   // \p{L}+
      return run_of(t, p, j, n, kL);
    case kN:   // \p{N}
      return j;
    case kO: {
      if (p[i] == '\'') {
        const size_t k = contraction(t, p, j, n);
        if (k) return k;
      }
      if (j < n && (prop_at(t, p, j, n, &l2) & 7) == kL) return run_of(t, p, j + l2, n, kL);   // [^\r\n\p{L}\p{N}]\p{L}+
      return nl_run(p, run_of(t, p, j, n, kO), n);   // [^\s\p{L}\p{N}]+[\r\n]*
    }
    case kSP: {
      if (j >= n) return n;
      const int c2 = prop_at(t, p, j, n, &l2) & 7;
      if (c2 == kL) return run_of(t, p, j + l2, n, kL);                  // " word"
      if (c2 == kO) return nl_run(p, run_of(t, p, j + l2, n, kO), n);   // " +=\n"
      return ws_piece(t, p, i, n);
    }
    case kWS: {
      if (j >= n) return n;
      if ((prop_at(t, p, j, n, &l2) & 7) == kL) return run_of(t, p, j + l2, n, kL);   // "\tword"
      return ws_piece(t, p, i, n);
    }
    default:   // CR / LF
      return ws_piece(t, p, i, n);
  }
}

// ---- BPE -----------------------------------------------------------------------------
constexpr uint32_t kNoRank = 0xFFFFFFFFu;

inline const MergeSlot* merge_of(const Tok& t, int32_t a, int32_t b) {
  const uint64_t key = ((uint64_t)(uint32_t)a << 32) | (uint32_t)b;
  const uint64_t mask = (1ull << t.mbits) - 1;
  uint64_t s = (key * 0x9E3779B97F4A7C15ull) >> (64 - t.mbits);
  while (true) {
    const MergeSlot& m = t.merges[s];
    if (m.key == key) return &m;
    if (m.key == ~0ull) return nullptr;
    s = (s + 1) & mask;
  }
}

inline int32_t direct_token(const Tok& t, const uint8_t* p, size_t n) {
  const uint64_t mask = (1ull << t.tbits) - 1;
  uint64_t s = hash_bytes(p, n) >> (64 - t.tbits);
  while (true) {
    const uint32_t e = t.tok_slots[s];
    if (!e) return -1;
    const uint32_t id = e - 1, a = t.tok_off[id], b = t.tok_off[id + 1];
    if (b - a == n && !memcmp(t.tok_bytes + a, p, n)) return (int32_t)id;
    s = (s + 1) & mask;
  }
}

inline void bpe(const Tok& t, const uint8_t* p, size_t n, std::vector<int32_t>& out) {
  std::vector<int32_t> sym(n);
  for (size_t i = 0; i < n; i++) sym[i] = t.byte_tok[p[i]];
  if (n <= 64) {   // short pieces: rescan for the best pair after every merge
    std::vector<const MergeSlot*> mg(n);
    size_t m = n;
    for (size_t i = 0; i + 1 < m; i++) mg[i] = merge_of(t, sym[i], sym[i + 1]);
    while (m > 1) {
      size_t bi = 0;
      uint32_t best = kNoRank;
      for (size_t i = 0; i + 1 < m; i++)
        if (mg[i] && mg[i]->rank < best) {
          best = mg[i]->rank;
          bi = i;
        }
      if (best == kNoRank) break;
      sym[bi] = (int32_t)mg[bi]->id;
      sym.erase(sym.begin() + bi + 1);
      mg.erase(mg.begin() + bi + 1);
      m--;
      if (bi > 0) mg[bi - 1] = merge_of(t, sym[bi - 1], sym[bi]);
      if (bi + 1 < m) mg[bi] = merge_of(t, sym[bi], sym[bi + 1]);
    }
    out.insert(out.end(), sym.begin(), sym.begin() + m);
    return;
  }
  // long pieces: a min-heap of (rank, position) over a linked list; entries whose pair has
  // changed since they were pushed are skipped when they come up
  std::vector<long> nxt(n), prv(n);
  for (size_t i = 0; i < n; i++) {
    prv[i] = (long)i - 1;
    nxt[i] = i + 1 < n ? (long)i + 1 : -1;
  }
  std::vector<uint64_t> heap;
  auto push = [&](uint64_t v) {
    heap.push_back(v);
    std::push_heap(heap.begin(), heap.end(), std::greater<uint64_t>());
  };
  for (size_t i = 0; i + 1 < n; i++) {
    const MergeSlot* m = merge_of(t, sym[i], sym[i + 1]);
    if (m) push(((uint64_t)m->rank << 32) | i);
  }
  while (!heap.empty()) {
    std::pop_heap(heap.begin(), heap.end(), std::greater<uint64_t>());
    const uint64_t top = heap.back();
    heap.pop_back();
    const uint32_t rank = (uint32_t)(top >> 32);
    const size_t pos = (size_t)(top & 0xFFFFFFFFu);
    if (sym[pos] < 0 || nxt[pos] < 0) continue;
    const size_t r = (size_t)nxt[pos];
    const MergeSlot* m = merge_of(t, sym[pos], sym[r]);
    if (!m || m->rank != rank) continue;
    sym[pos] = (int32_t)m->id;
    sym[r] = -1;
    nxt[pos] = nxt[r];
    if (nxt[r] >= 0) prv[nxt[r]] = (long)pos;
    if (prv[pos] >= 0) {
      const MergeSlot* a = merge_of(t, sym[prv[pos]], sym[pos]);
      if (a) push(((uint64_t)a->rank << 32) | (uint64_t)prv[pos]);
    }
    if (nxt[pos] >= 0) {
      const MergeSlot* b = merge_of(t, sym[pos], sym[nxt[pos]]);
      if (b) push(((uint64_t)b->rank << 32) | pos);
    }
  }
  for (long i = 0; i >= 0; i = nxt[i]) out.push_back(sym[i]);
}

inline void emit_piece(const Tok& t, const uint8_t* p, size_t n, std::vector<int32_t>& out) {
  if (n == 1) {
    out.push_back(t.byte_tok[p[0]]);
    return;
  }
  if ((int64_t)n <= t.max_len) {
    const int32_t id = direct_token(t, p, n);
    if (id >= 0) {
      out.push_back(id);
      return;
    }
  }
  bpe(t, p, n, out);
}

// One segment without added tokens: NFC, pieces, tokens.
inline void encode_segment(const Tok& t, const uint8_t* p, size_t n, std::vector<int32_t>& out) {
  std::string norm;
  if (needs_nfc(t, p, n)) {
    nfc(t, p, n, norm);
    p = (const uint8_t*)norm.data();
    n = norm.size();
  }
  for (size_t i = 0; i < n;) {
    const size_t j = piece_end(t, p, i, n);
    emit_piece(t, p + i, j - i, out);
    i = j;
  }
}

// The longest added token at p[q], or -1 (and its length).
inline int32_t added_at(const Tok& t, const uint8_t* p, size_t q, size_t n, size_t* len) {
  int32_t best = -1;
  size_t bl = 0;
  for (int64_t k = 0; k < t.n_added; k++) {
    const uint32_t id = t.added[3 * k], off = t.added[3 * k + 1], l = t.added[3 * k + 2];
    if (l == 0 || l <= bl || q + l > n) continue;
    if (!memcmp(t.added_bytes + off, p + q, l)) {
      best = (int32_t)id;
      bl = l;
    }
  }
  *len = bl;
  return best;
}

inline void encode(const Tok& t, const uint8_t* p, size_t n, bool specials, std::vector<int32_t>& out) {
  if (!specials) {
    encode_segment(t, p, n, out);
    return;
  }
  size_t seg = 0;
  for (size_t q = 0; q < n;) {
    size_t l = 0;
    const int32_t id = t.first_byte[p[q]] ? added_at(t, p, q, n, &l) : -1;
    if (id < 0) {
      q++;
      continue;
    }
    if (q > seg) encode_segment(t, p + seg, q - seg, out);
    out.push_back(id);
    q += l;
    seg = q;
  }
  if (seg < n) encode_segment(t, p + seg, n - seg, out);
}

// Maps and checks a compiled file; "" on success, else the reason.
inline std::string open(const char* path, Tok& t) {
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return std::string("cannot open ") + path;
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return std::string("cannot stat ") + path;
  }
  t.size = (size_t)st.st_size;
  if (t.size < kHdrWords * 8) {
    ::close(fd);
    return std::string(path) + ": too small for a tokenizer file";
  }
  void* m = mmap(nullptr, t.size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return std::string("mmap failed for ") + path;
  t.map = m;
  const uint64_t* h = (const uint64_t*)m;
  const uint8_t* base = (const uint8_t*)m;
  if (h[0] != kMagic || h[1] != t.size) return std::string(path) + ": not an ILTK1 tokenizer file (compile it with python -m instantllm_amd.tokenizer compile)";
  t.n_total = (int64_t)h[2];
  t.n_vocab = (int64_t)h[3];
  t.n_added = (int64_t)h[5];
  t.max_len = (int64_t)h[6];
  t.tbits = (int)h[7];
  t.mbits = (int)h[8];
  t.im_start = (int32_t)(int64_t)h[9];
  t.im_end = (int32_t)(int64_t)h[10];
  t.eot = (int32_t)(int64_t)h[11];
  t.n_blocks = (int64_t)h[12];
  t.n_dec = (int64_t)h[13];
  t.n_ddata = (int64_t)h[14];
  t.n_comp = (int64_t)h[15];
  if (t.n_total < 256 || t.n_total > (1 << 24) || t.tbits < 4 || t.tbits > 30 || t.mbits < 4 || t.mbits > 30 || t.n_added < 0 ||
      t.n_added > 4096 || t.n_blocks < 1 || t.n_blocks > 4352)
    return std::string(path) + ": header out of range";
  // every section inside the file, 8-byte aligned, ordered and large enough
  const uint64_t need[14] = {(uint64_t)(t.n_total + 1) * 4, 0, 1024, 4ull << t.tbits, 16ull << t.mbits,
                             (uint64_t)t.n_added * 12, 0, 0x1100 * 2, (uint64_t)t.n_blocks * 512, (uint64_t)t.n_dec * 4,
                             (uint64_t)t.n_dec * 4, (uint64_t)t.n_ddata * 4, (uint64_t)t.n_comp * 8, (uint64_t)t.n_comp * 4};
  for (int k = 0; k < 14; k++) {
    const uint64_t a = h[20 + k], b = k + 1 < 14 ? h[21 + k] : t.size;
    if (a % 8 || a < kHdrWords * 8 || b > t.size || a > b || b - a < need[k]) return std::string(path) + ": section out of range";
  }
  t.tok_off = (const uint32_t*)(base + h[20]);
  t.tok_bytes = base + h[21];
  if (t.tok_off[0] != 0 || h[21] + t.tok_off[t.n_total] > h[22]) return std::string(path) + ": token bytes out of range";
  for (int64_t i = 0; i < t.n_total; i++)
    if (t.tok_off[i + 1] < t.tok_off[i]) return std::string(path) + ": token offsets not ordered";
  t.byte_tok = (const int32_t*)(base + h[22]);
  t.tok_slots = (const uint32_t*)(base + h[23]);
  t.merges = (const MergeSlot*)(base + h[24]);
  t.added = (const uint32_t*)(base + h[25]);
  t.added_bytes = base + h[26];
  t.uni_top = (const uint16_t*)(base + h[27]);
  t.uni_blocks = (const uint16_t*)(base + h[28]);
  t.dkeys = (const uint32_t*)(base + h[29]);
  t.dvals = (const uint32_t*)(base + h[30]);
  t.ddata = (const uint32_t*)(base + h[31]);
  t.ckeys = (const uint64_t*)(base + h[32]);
  t.cvals = (const uint32_t*)(base + h[33]);
  for (int b = 0; b < 256; b++)
    if (t.byte_tok[b] < 0 || t.byte_tok[b] >= t.n_total) return std::string(path) + ": byte token out of range";
  for (int k = 0; k < 0x1100; k++)
    if (t.uni_top[k] >= t.n_blocks) return std::string(path) + ": Unicode table out of range";
  for (int64_t k = 0; k < t.n_dec; k++)
    if ((t.dvals[k] >> 8) + (t.dvals[k] & 255) > (uint64_t)t.n_ddata) return std::string(path) + ": decomposition out of range";
  // the code points NFC may write: scalar values only, so that its output is UTF-8
  auto scalar = [](uint32_t c) { return c < 0x110000 && (c < 0xD800 || c > 0xDFFF); };
  for (int64_t k = 0; k < t.n_ddata; k++)
    if (!scalar(t.ddata[k])) return std::string(path) + ": decomposition holds a non-scalar code point";
  for (int64_t k = 0; k < t.n_comp; k++)
    if (!scalar(t.cvals[k])) return std::string(path) + ": composition holds a non-scalar code point";
  const uint64_t abytes = h[27] - h[26];
  for (int64_t k = 0; k < t.n_added; k++) {
    const uint32_t id = t.added[3 * k], off = t.added[3 * k + 1], l = t.added[3 * k + 2];
    if (id >= t.n_total || (uint64_t)off + l > abytes) return std::string(path) + ": added token out of range";
    if (l) t.first_byte[t.added_bytes[off]] = true;
  }
  for (uint64_t s = 0; s < (1ull << t.tbits); s++)
    if (t.tok_slots[s] > (uint64_t)t.n_total) return std::string(path) + ": token table out of range";
  for (uint64_t s = 0; s < (1ull << t.mbits); s++)
    if (t.merges[s].key != ~0ull && t.merges[s].id >= t.n_total) return std::string(path) + ": merge table out of range";
  // the chat template: S "system\n" {system} E "\n" S "user\n" {user} E "\n" S "assistant\n"
  if (t.im_start >= 0 && t.im_end >= 0) {
    std::string s, e;
    for (int64_t k = 0; k < t.n_added; k++) {
      const uint32_t id = t.added[3 * k], off = t.added[3 * k + 1], l = t.added[3 * k + 2];
      if ((int32_t)id == t.im_start) s.assign((const char*)t.added_bytes + off, l);
      if ((int32_t)id == t.im_end) e.assign((const char*)t.added_bytes + off, l);
    }
    t.chat0 = s + "system\n";
    t.chat1 = e + "\n" + s + "user\n";
    t.chat2 = e + "\n" + s + "assistant\n";
  }
  return std::string();
}

}  // namespace iltk
