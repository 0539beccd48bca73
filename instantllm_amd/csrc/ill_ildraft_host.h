// Host side of the learned drafter: ILDRAFT1 table load and the per-request context.
//
// Reference: ILDraft.swift (init :38-84, prepare :110-208); format tools/draft/ildraft.py:16-53.
// The request context is prepared on the CPU once per request (TF-IDF neighbours, copy
// candidates, prompt-word associations) and copied to the device, where the drafting kernel
// reads it (ill_ildraft.h).
#pragma once
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "ill_ildraft.h"

namespace illd {

constexpr int32_t kTail[5] = {151645, 198, 151644, 77091, 198};

inline uint64_t fnv1a64(const uint8_t* b, size_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; i++) {
    h ^= b[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

// Distinct runs of [a-z0-9] of the ASCII-lowercased UTF-8 text, first appearance first.
inline std::vector<std::string> prompt_words(const char* text) {
  std::vector<std::string> out;
  std::set<std::string> seen;
  std::string cur;
  for (const char* p = text;; ++p) {
    unsigned char c = (unsigned char)*p;
    if (c >= 'A' && c <= 'Z') c += 32;
    if ((c >= 'a' && c <= 'z') || (c >= '0' && c <= '9')) {
      cur.push_back((char)c);
      continue;
    }
    if (!cur.empty()) {
      if (seen.insert(cur).second) out.push_back(cur);
      cur.clear();
    }
    if (!*p) break;
  }
  return out;
}

// Runs of [A-Za-z0-9_.\-/~:@] of the text, in order (space-variant candidates).
inline std::vector<std::string> spacevar_words(const char* text) {
  std::vector<std::string> out;
  std::string cur;
  for (const char* p = text;; ++p) {
    const unsigned char c = (unsigned char)*p;
    const bool ok = (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_' ||
                    c == '.' || c == '-' || c == '/' || c == '~' || c == ':' || c == '@';
    if (ok && c) {
      cur.push_back((char)c);
      continue;
    }
    if (!cur.empty()) {
      out.push_back(cur);
      cur.clear();
    }
    if (!*p) break;
  }
  return out;
}

struct Section {
  uint32_t cnt = 0;
  uint64_t off = 0;
  bool present = false;
};

struct Table {
  std::vector<uint8_t> blob;
  std::map<std::string, Section> sec;
  uint32_t N = 0, M = 0, KNB = 0, MAXM = 0, F = 0, H = 0, D = 0, flags = 0;
  std::vector<uint8_t> tflg;     // [ILD_VOCAB]
  std::vector<double> doc_score;
  std::vector<int32_t> touched;
  IllDraftReq req{};

  template <typename T>
  T at(uint64_t off) const {
    T v;
    memcpy(&v, blob.data() + off, sizeof v);
    return v;
  }
  const Section& s(const char* tag) const { return sec.at(tag); }

  // Index of key in a section of ascending u64 keys, or -1.
  int find64(const char* tag, uint64_t key) const {
    const Section& x = s(tag);
    int lo = 0, hi = (int)x.cnt;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (at<uint64_t>(x.off + 8ull * mid) < key) lo = mid + 1;
      else hi = mid;
    }
    return lo < (int)x.cnt && at<uint64_t>(x.off + 8ull * lo) == key ? lo : -1;
  }
  // Copy rate of a prompt token (CPTK {u32 token, f32 rate}, ascending; default 0.2).
  float prop(int32_t tok) const {
    const Section& x = s("CPTK");
    int lo = 0, hi = (int)x.cnt;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (at<uint32_t>(x.off + 8ull * mid) < (uint32_t)tok) lo = mid + 1;
      else hi = mid;
    }
    return lo < (int)x.cnt && at<uint32_t>(x.off + 8ull * lo) == (uint32_t)tok ? at<float>(x.off + 8ull * lo + 4) : 0.2f;
  }
};

// Parses and checks a table file (ILDraft.swift:38-71); returns an empty string or the error.
inline std::string load(Table& t, const char* path) {
  FILE* f = fopen(path, "rb");
  if (!f) return std::string("cannot read ") + path;
  fseek(f, 0, SEEK_END);
  const long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  t.blob.resize(n > 0 ? (size_t)n : 0);
  const size_t got = n > 0 ? fread(t.blob.data(), 1, (size_t)n, f) : 0;
  fclose(f);
  if (n < 64 || got != (size_t)n) return std::string("cannot read ") + path;
  uint32_t h[16];
  memcpy(h, t.blob.data(), 64);
  if (memcmp(t.blob.data(), "ILDRAFT1", 8) != 0 || h[2] != 1) return std::string(path) + ": not an ILDRAFT1 table";
  const uint32_t nsec = h[3];
  t.N = h[4];
  t.M = h[5];
  t.KNB = h[6];
  t.MAXM = h[7];
  t.F = h[8];
  t.H = h[9];
  t.D = h[11];
  t.flags = h[12];
  if (t.F != ILD_NF || t.N > 6 || t.M > 7 || t.KNB > ILD_MAXNB || t.MAXM > 12 || t.H > ILD_MAXH || t.H < 1)
    return std::string(path) + ": unsupported drafter config";
  if (64ull + 16ull * nsec > t.blob.size()) return std::string(path) + ": truncated section directory";
  static const std::map<std::string, int> esize = {
      {"NGKY", 8}, {"NGVL", 8}, {"NGNX", 8}, {"WDKY", 8}, {"WDVL", 12}, {"POST", 4}, {"DNRM", 4}, {"SQOF", 4},
      {"SQTK", 4}, {"CPTK", 8}, {"CPC1", 8}, {"CPC2", 16}, {"ASWK", 8}, {"ASWV", 8}, {"ASTK", 8}, {"TFLS", 8},
      {"MLP0", 4}, {"PTXO", 4}, {"PTXB", 1}, {"TFLG", 1}};
  for (uint32_t i = 0; i < nsec; i++) {
    const uint8_t* b = t.blob.data() + 64 + 16 * i;
    std::string tag((const char*)b, 4);
    Section x;
    memcpy(&x.cnt, b + 4, 4);
    memcpy(&x.off, b + 8, 8);
    x.present = true;
    const auto it = esize.find(tag);
    const uint64_t bytes = (uint64_t)x.cnt * (it == esize.end() ? 1 : it->second);
    if (x.off > t.blob.size() || bytes > t.blob.size() - x.off) return std::string(path) + ": section " + tag + " out of range";
    t.sec[tag] = x;
  }
  for (const char* tag : {"NGKY", "NGVL", "NGNX", "WDKY", "WDVL", "POST", "DNRM", "SQOF", "SQTK", "CPTK", "CPC1", "CPC2",
                          "TFLS", "MLP0"})
    if (!t.sec.count(tag)) return std::string(path) + ": missing section " + tag;
  if (t.s("NGVL").cnt != t.s("NGKY").cnt || t.s("WDVL").cnt != t.s("WDKY").cnt || t.s("DNRM").cnt != t.D ||
      t.s("SQOF").cnt != t.D + 1)
    return std::string(path) + ": inconsistent section sizes";
  if (t.s("MLP0").cnt != t.H * ILD_NF + 2 * t.H + 1 + ILD_NF) return std::string(path) + ": scorer size mismatch";
  if (t.s("NGKY").off % 8 || t.s("NGVL").off % 8 || t.s("NGNX").off % 8 || t.s("CPC1").off % 8 || t.s("CPC2").off % 8 ||
      t.s("MLP0").off % 4)
    return std::string(path) + ": misaligned section";
  // the n-gram continuations and posting / sequence offsets must stay inside their sections
  const Section& vl = t.s("NGVL");
  for (uint32_t i = 0; i < vl.cnt; i++) {
    const uint32_t fn = t.at<uint32_t>(vl.off + 8ull * i + 4);
    if ((fn >> 3) + (fn & 7) > t.s("NGNX").cnt) return std::string(path) + ": n-gram entry out of range";
  }
  const Section& wv = t.s("WDVL");
  for (uint32_t i = 0; i < wv.cnt; i++) {
    const uint32_t first = t.at<uint32_t>(wv.off + 12ull * i + 4), n = t.at<uint32_t>(wv.off + 12ull * i + 8);
    if ((uint64_t)first + n > t.s("POST").cnt) return std::string(path) + ": posting list out of range";
  }
  for (uint32_t i = 0; i < t.s("POST").cnt; i++)
    if (t.at<uint32_t>(t.s("POST").off + 4ull * i) >= t.D) return std::string(path) + ": posting out of range";
  for (uint32_t i = 0; i <= t.D; i++) {
    const uint32_t o = t.at<uint32_t>(t.s("SQOF").off + 4ull * i);
    if (o > t.s("SQTK").cnt || (i > 0 && o < t.at<uint32_t>(t.s("SQOF").off + 4ull * (i - 1))))
      return std::string(path) + ": sequence offsets out of range";
  }
  if (t.flags & 1) {
    for (const char* tag : {"ASWK", "ASWV", "ASTK"})
      if (!t.sec.count(tag)) return std::string(path) + ": missing section " + tag;
    const Section& av = t.s("ASWV");
    for (uint32_t i = 0; i < av.cnt; i++) {
      const uint32_t first = t.at<uint32_t>(av.off + 8ull * i), n = t.at<uint32_t>(av.off + 8ull * i + 4);
      if ((uint64_t)first + n > t.s("ASTK").cnt) return std::string(path) + ": association list out of range";
    }
  }
  t.tflg.assign(ILD_VOCAB, 0);
  const Section& tf = t.s("TFLS");
  for (uint32_t i = 0; i < tf.cnt; i++) {
    const uint32_t tok = t.at<uint32_t>(tf.off + 8ull * i), v = t.at<uint32_t>(tf.off + 8ull * i + 4);
    if (tok < ILD_VOCAB) t.tflg[tok] = (uint8_t)v;
  }
  t.doc_score.assign(t.D, 0.0);
  t.touched.clear();
  return std::string();
}

// The first id of encode(text) through the caller's tokenizer callback, or -1.
typedef int (*EncodeFn)(void* user, const char* text, int32_t* ids, int cap);

// Prepares the request context (ILDraft.swift:110-208): `prompt` = the user prompt's ids
// inside the chat template, `text` = the user prompt, `enc` = the tokenizer (may be null:
// no space-variant candidates).
inline void prepare(Table& t, const int32_t* prompt, int n, const char* text, EncodeFn enc, void* user) {
  IllDraftReq& r = t.req;
  memset(&r, 0, sizeof r);
  const int np = std::min(n, ILD_MAXP);
  r.np = np;
  std::set<int32_t> pset;
  for (int i = 0; i < np; i++) {
    r.P[i] = prompt[i];
    pset.insert(prompt[i]);
  }
  for (int i = 0; i < np; i++) r.pprop[i] = t.prop(r.P[i]);
  // neighbours: TF-IDF cosine over the prompt words, top KNB by (score desc, doc asc), in
  // float64 so the order matches the Python drafter's
  const std::vector<std::string> words = prompt_words(text ? text : "");
  for (int32_t d : t.touched) t.doc_score[d] = 0.0;
  t.touched.clear();
  double q2 = 0.0;
  const Section& wv = t.s("WDVL");
  const Section& po = t.s("POST");
  for (const std::string& w : words) {
    const int k = t.find64("WDKY", fnv1a64((const uint8_t*)w.data(), w.size()));
    if (k < 0) continue;
    const double idf = (double)t.at<float>(wv.off + 12ull * k);
    const uint32_t first = t.at<uint32_t>(wv.off + 12ull * k + 4), cnt = t.at<uint32_t>(wv.off + 12ull * k + 8);
    const double w2 = idf * idf;
    q2 += w2;
    for (uint32_t j = 0; j < cnt; j++) {
      const uint32_t doc = t.at<uint32_t>(po.off + 4ull * (first + j));
      if (t.doc_score[doc] == 0.0) t.touched.push_back((int32_t)doc);
      t.doc_score[doc] += w2;
    }
  }
  const double qn = q2 > 0 ? std::sqrt(q2) : 1.0;
  std::vector<std::pair<double, int32_t>> ranked;
  ranked.reserve(t.touched.size());
  for (int32_t d : t.touched)
    ranked.emplace_back(t.doc_score[d] / (qn * (double)t.at<float>(t.s("DNRM").off + 4ull * d)), d);
  std::sort(ranked.begin(), ranked.end(), [](const std::pair<double, int32_t>& x, const std::pair<double, int32_t>& y) {
    return x.first != y.first ? x.first > y.first : x.second < y.second;
  });
  const int nb = std::min<int>(std::min<int>((int)t.KNB, ILD_MAXNB), (int)ranked.size());
  r.nnb = nb;
  int pos = 0;
  const Section& sqof = t.s("SQOF");
  const Section& sqtk = t.s("SQTK");
  for (int i = 0; i < nb; i++) {
    const int32_t d = ranked[i].second;
    r.nbScore[i] = (float)ranked[i].first;
    r.nbOff[i] = pos;
    int len = 0;
    for (int k = 0; k < 5 && len < ILD_NBSEQ; k++, len++) r.nbTok[pos++] = kTail[k];
    const uint32_t a0 = t.at<uint32_t>(sqof.off + 4ull * d), a1 = t.at<uint32_t>(sqof.off + 4ull * (d + 1));
    for (uint32_t j = a0; j < a1 && len < ILD_NBSEQ; j++, len++) r.nbTok[pos++] = (int32_t)t.at<uint32_t>(sqtk.off + 4ull * j);
  }
  r.nbOff[nb] = pos;
  // copy candidates: prompt ids and the first id of " word" for each space-variant word
  std::set<int32_t> cand = pset;
  if (enc) {
    int32_t ids[8];
    for (const std::string& w : spacevar_words(text ? text : "")) {
      const std::string s = " " + w;
      const int got = enc(user, s.c_str(), ids, 8);
      if (got > 0 && !pset.count(ids[0])) cand.insert(ids[0]);
    }
  }
  int nc = 0;
  for (int32_t x : cand) {
    if (nc >= ILD_MAXCOPY) break;
    const bool inp = pset.count(x) != 0;
    r.copyTok[nc] = x;
    r.copyInP[nc] = inp ? 1 : 0;
    const float pt = inp ? t.prop(x) : 0.3f;
    r.copyPt[nc] = pt;
    r.copyF33[nc] = (float)std::log((double)(pt / (1.f - pt))) / 4.f;
    nc++;
  }
  r.ncopy = nc;
  // prompt-word -> output-token associations: (max ln-lift, number of words)
  std::map<int32_t, std::pair<float, int32_t>> as;
  if ((t.flags & 1) && t.sec.count("ASWK")) {
    const Section& av = t.s("ASWV");
    const Section& at = t.s("ASTK");
    for (const std::string& w : words) {
      const int k = t.find64("ASWK", fnv1a64((const uint8_t*)w.data(), w.size()));
      if (k < 0) continue;
      const uint32_t first = t.at<uint32_t>(av.off + 8ull * k), cnt = t.at<uint32_t>(av.off + 8ull * k + 4);
      for (uint32_t j = 0; j < cnt; j++) {
        const int32_t tok = (int32_t)t.at<uint32_t>(at.off + 8ull * (first + j));
        const float ll = t.at<float>(at.off + 8ull * (first + j) + 4);
        auto it = as.find(tok);
        if (it == as.end()) as[tok] = {ll, 1};
        else it->second = {std::max(it->second.first, ll), it->second.second + 1};
      }
    }
  }
  int na = 0;
  for (const auto& e : as) {
    if (na >= ILD_MAXAS) break;
    r.asTok[na] = e.first;
    r.asMax[na] = e.second.first;
    r.asCnt[na] = e.second.second;
    na++;
  }
  r.nas = na;
}

// Hash indexes of the three searched sections (the drafting kernel's ild_hfind): for each, a
// power of two of 32-byte slots, at least twice the section's entries, each used slot
// {key lo, key hi, 1, v0, v1, 0, 0, 0}: NGKY keys with their NGVL entry (total, count and
// first continuation), CPC1 / CPC2 keys with their rate. Entries are inserted in section
// order and a repeated key keeps its first entry. Offsets (bytes into `out`, 32-aligned) and
// the bit counts are returned in the order NGKY, CPC1, CPC2.
struct HashIndex {
  std::vector<uint8_t> bytes;
  uint64_t off[3];
  uint32_t bits[3];
};
inline uint32_t hash_slot(uint64_t key, uint32_t bits) { return (uint32_t)((key * 0x9E3779B97F4A7C15ull) >> (64 - bits)); }
inline HashIndex build_index(const Table& t) {
  HashIndex hx;
  const char* tags[3] = {"NGKY", "CPC1", "CPC2"};
  for (int k = 0; k < 3; k++) {
    const Section& x = t.s(tags[k]);
    uint32_t bits = 4;
    while ((1ull << bits) < 2ull * x.cnt) bits++;
    if (bits > 28) {   // 2^28 slots (8 GiB) at most: a larger section is refused by the loader
      hx.bits[k] = 0;
      hx.bytes.clear();
      return hx;
    }
    const uint64_t nslot = 1ull << bits;
    hx.off[k] = hx.bytes.size();
    hx.bits[k] = bits;
    hx.bytes.resize(hx.bytes.size() + 32 * nslot, 0);
    uint32_t* sl = (uint32_t*)(hx.bytes.data() + hx.off[k]);
    for (uint64_t i = 0; i < x.cnt; i++) {
      uint64_t key;
      uint32_t v0, v1 = 0;
      if (k == 0) {
        key = t.at<uint64_t>(x.off + 8 * i);
        v0 = t.at<uint32_t>(t.s("NGVL").off + 8 * i);
        v1 = t.at<uint32_t>(t.s("NGVL").off + 8 * i + 4);
      } else if (k == 1) {
        key = t.at<uint32_t>(x.off + 8 * i);
        v0 = t.at<uint32_t>(x.off + 8 * i + 4);
      } else {
        key = t.at<uint64_t>(x.off + 16 * i);
        v0 = t.at<uint32_t>(x.off + 16 * i + 8);
      }
      uint32_t hs = hash_slot(key, bits);
      for (;;) {
        uint32_t* e = sl + 8 * (uint64_t)hs;
        if (e[2] == 0) {
          e[0] = (uint32_t)key;
          e[1] = (uint32_t)(key >> 32);
          e[2] = 1;
          e[3] = v0;
          e[4] = v1;
          break;
        }
        if (((uint64_t)e[1] << 32 | e[0]) == key) break;   // a repeated key keeps its first entry
        hs = (hs + 1) & (uint32_t)(nslot - 1);
      }
    }
  }
  return hx;
}

// The device view of a table uploaded to `dtab` (DraftMeta, ILDraft.swift:73-80), its hash
// indexes uploaded to `dhash` (HashIndex::bytes).
inline IllDraftArgs device_args(const Table& t, const uint8_t* dtab, const uint8_t* dtflg, const IllDraftReq* dreq,
                                const HashIndex& hx, const uint8_t* dhash) {
  IllDraftArgs a{};
  a.tab = dtab;
  a.tflg = dtflg;
  a.req = dreq;
  a.ngky = t.s("NGKY").off;
  a.ngvl = t.s("NGVL").off;
  a.ngnx = t.s("NGNX").off;
  a.cpc1 = t.s("CPC1").off;
  a.cpc2 = t.s("CPC2").off;
  a.mlp = t.s("MLP0").off;
  a.n_ngky = (int32_t)t.s("NGKY").cnt;
  a.n_cpc1 = (int32_t)t.s("CPC1").cnt;
  a.n_cpc2 = (int32_t)t.s("CPC2").cnt;
  a.N = (int32_t)t.N;
  a.M = (int32_t)t.M;
  a.MAXM = (int32_t)t.MAXM;
  a.H = (int32_t)t.H;
  a.hng = (const uint4*)(dhash + hx.off[0]);
  a.hc1 = (const uint4*)(dhash + hx.off[1]);
  a.hc2 = (const uint4*)(dhash + hx.off[2]);
  a.bng = hx.bits[0];
  a.bc1 = hx.bits[1];
  a.bc2 = hx.bits[2];
  return a;
}

}  // namespace illd
