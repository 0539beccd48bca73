// Learned speculative drafter: ILDRAFT1 tables, per-request context and the drafting kernel.
//
// Reference: tools/draft/ildraft.py (the specification and table format, :16-53), its
// engine port ILDraft.swift (table load :38-84, request context :110-208) and k_ildraft
// (Shaders.swift:421-872). After a speculative commit that did not stop, the drafting
// kernel proposes the next pass's rows: a chain of up to T - 1 tokens or a best-first tree
// of up to tree_b tokens, each step scoring the candidates of the n-gram table,
// self-repetition, prompt lookup, the request's TF-IDF neighbours' outputs and the copy
// candidates with 53 features and a small MLP.
//
// GPU shape: one workgroup of 1024 threads (16 waves). Per drafted token the waves split
// the sources (wave 0 the six n-gram orders, ten lanes each, through a hash index of the
// table's sorted keys built at load, 1 self-repetition, 2 prompt lookup, 3 the copy
// context through the same kind of index, 4-11 two neighbours each),
// then two threads per distinct candidate (in waves 0-7 and 8-15) write its 53 features to
// LDS, and the scorer runs with one lane per hidden unit (16 or 32 lanes per candidate),
// the hidden unit's and the linear term's sums advancing together. The candidate
// set is deduplicated through an LDS hash set, so its order in memory is arbitrary: every
// decision depends on the set only (argmax by (score desc, token asc); the tree's top 8 by
// the same order; the softmax normaliser summed in float64 and rounded to float32).
#pragma once
#include "ill_pass.h"

#define ILD_MAXP 256
#define ILD_MAXCOPY 256
#define ILD_MAXNB 16
#define ILD_NBSEQ 80
#define ILD_MAXAS 1024
#define ILD_NF 53
#define ILD_FS 56                // LDS row stride of the feature rows (16-byte rows for vector reads)
#define ILD_MAXH 32
#define ILD_W1S 57               // LDS row stride of W1 (odd: the lanes of 16 hidden units hit distinct banks)
#define ILD_THREADS 1024
#define ILD_NRAW (85 + ILD_MAXCOPY)
#define ILD_HASH 1024
#define ILD_HEAP 128
#define ILD_OB (ILL_OB_MAX + ILL_MAXT)
#define ILD_VOCAB 151936
#define ILD_LG1P 512

// The per-request context (DraftReq, ILDraft.swift:20-35 / Shaders.swift:432-447), with the
// request-constant copy features computed on the host: pprop[i] = rate of P[i] (CPTK,
// default 0.2), copyPt[i] = rate of copyTok[i] if it is a prompt id, else 0.3, copyF33[i]
// its feature 33 (the logit over 4).
struct IllDraftReq {
  int32_t np, ncopy, nnb, nas;
  int32_t P[ILD_MAXP];
  float pprop[ILD_MAXP];
  int32_t copyTok[ILD_MAXCOPY];   // ascending
  int32_t copyInP[ILD_MAXCOPY];
  float copyPt[ILD_MAXCOPY];
  float copyF33[ILD_MAXCOPY];     // ln(pt / (1 - pt)) / 4 of copyPt (float32 ops, ln in float64)
  float nbScore[ILD_MAXNB];
  int32_t nbOff[ILD_MAXNB + 1];
  int32_t pad[3];
  int32_t nbTok[ILD_MAXNB * ILD_NBSEQ];
  int32_t asTok[ILD_MAXAS];       // ascending
  float asMax[ILD_MAXAS];
  int32_t asCnt[ILD_MAXAS];
};

// Device view of a loaded table (DraftMeta, ILDraft.swift:73-80).
struct IllDraftArgs {
  const uint8_t* tab;        // the table file as is
  const uint8_t* tflg;       // [ILD_VOCAB] '`' count (bits 0-2), newline (bit 3)
  const IllDraftReq* req;
  uint64_t ngky, ngvl, ngnx, cpc1, cpc2, mlp;   // byte offsets of the sections
  int32_t n_ngky, n_cpc1, n_cpc2;
  int32_t N, M, MAXM, H;
  // Hash indexes of NGKY, CPC1 and CPC2 built when the table loads (ild_hfind): 2^bits
  // slots of 32 B each, a slot holding the key and the entry's values, so a lookup is one
  // round trip to memory instead of the sorted sections' search
  const uint4* hng;
  const uint4* hc1;
  const uint4* hc2;
  uint32_t bng, bc1, bc2;
};

__device__ __forceinline__ int ild_tail(int i) {
  return i == 0 ? 151645 : (i == 1 ? 198 : (i == 2 ? 151644 : (i == 3 ? 77091 : 198)));
}

struct IldLds {
  IllDraftReq R;
  float w1[ILD_MAXH * ILD_W1S];
  float b1[ILD_MAXH], w2[ILD_MAXH];
  alignas(16) float wl[ILD_W1S];
  float b2;
  float lg1p[ILD_LG1P];      // ln(1 + c) of the counts c < ILD_LG1P
  int ob[ILD_OB];
  int used[ILD_HASH];        // tokens of the output window (hash set)
  int cset[ILD_HASH];        // candidates (hash set)
  int uniq[ILD_NRAW];
  uint64_t ckey[ILD_NRAW];
  float csc[ILD_NRAW];
  int ctf[ILD_NRAW];         // '`' count of each candidate
  alignas(16) float F[ILD_NRAW * ILD_FS];   // feature rows (ILD_NF used of ILD_FS)
  int pm[ILD_MAXP];
  // phase A results
  int dist_tot[8], dist_cnt[8], top_tok[8][8], top_cnt[8][8];
  int s_long, s_supp3, s_supp10, s_toplong, s_entlow;
  int self_n, self_tok;
  int pr_n, pr_cnt, pr_tok[32];
  int vote_tok[ILD_MAXNB], vote_n[ILD_MAXNB];
  float c1, c2;
  int firstun;
  // drafting state (thread 0 writes between iterations)
  int go, depth, nd, rows, erow, ticks, ticks0, nu;
  int next_rows[ILL_MAXT];
  int tr_par[ILL_MAXT], tr_tok[ILL_MAXT], tr_dep[ILL_MAXT];
  uint32_t tr_anc[ILL_MAXT];
  float tr_cum[ILL_MAXT];
  int tr_tf[ILL_MAXT];
  float h_cum[ILD_HEAP];
  int h_par[ILD_HEAP], h_tok[ILD_HEAP], h_ord[ILD_HEAP], h_tf[ILD_HEAP];
  int h_n, h_ctr;
  int tk_tok[8], tk_tf[8];
  float tk_e[8];
  uint64_t red64[ILD_THREADS / 64];
  double redd[ILD_THREADS / 64];
  int best_tf;
  int flag;
};

static_assert(ILD_HASH == ILD_THREADS, "the hash sets are cleared one slot per thread");
static_assert(ILD_FS % 4 == 0 && ILD_FS >= ILD_NF && ILD_W1S >= ILD_FS, "vector reads of feature rows and linear weights");
static_assert(sizeof(IllDraftReq) % 16 == 0, "the request is staged in 16-byte units");

__device__ __forceinline__ uint32_t ild_hash(int key) { return ((uint32_t)key * 2654435761u) >> 22; }

// Insert into an LDS hash set (-1 = empty); true when the key was not there before.
__device__ __forceinline__ bool ild_insert(int* set, int key) {
  uint32_t s = ild_hash(key);
  for (int probe = 0; probe < ILD_HASH; probe++) {
    const int old = atomicCAS(set + s, -1, key);
    if (old == -1) return true;
    if (old == key) return false;
    s = (s + 1) & (ILD_HASH - 1);
  }
  return false;
}

__device__ __forceinline__ bool ild_has(const int* set, int key) {
  uint32_t s = ild_hash(key);
  for (int probe = 0; probe < ILD_HASH; probe++) {
    const int v = set[s];
    if (v == key) return true;
    if (v == -1) return false;
    s = (s + 1) & (ILD_HASH - 1);
  }
  return false;
}

// Index of key in an ascending LDS array of n ints, or -1.
__device__ __forceinline__ int ild_bsearch(const int* a, int n, int key) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  return lo < n && a[lo] == key ? lo : -1;
}

__device__ __forceinline__ void ild_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t ild_wave_max(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ uint64_t ild_max64(uint64_t v, int width) {
  for (int off = width >> 1; off >= 1; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

// Open-addressing lookup in an index of 2^bits slots {key (u64), used, v0, v1, -, -, -}
// built by illd::build_index (multiplicative hash, linear probing; the lowest entry of a key
// when a section repeats it, as a lower-bound search finds). True with the entry's values.
__device__ __forceinline__ uint64_t ild_hslot(uint64_t key, uint32_t bits) { return (key * 0x9E3779B97F4A7C15ull) >> (64 - bits); }
__device__ bool ild_hfind(const uint4* slots, uint32_t bits, uint64_t key, uint32_t& v0, uint32_t& v1) {
  const uint32_t mask = (1u << bits) - 1u;
  uint32_t h = (uint32_t)ild_hslot(key, bits);
  for (uint32_t probe = 0; probe <= mask; probe++) {
    const uint4 a = slots[2 * h], b = slots[2 * h + 1];
    if (a.z == 0u) return false;
    if ((((uint64_t)a.y << 32) | a.x) == key) {
      v0 = a.w;
      v1 = b.x;
      return true;
    }
    h = (h + 1u) & mask;
  }
  return false;
}

// sc + W2[hh] relu(a_hh) for hh = 0, 1, ..., H - 1 in that order, a_hh being lane hh's value
// of this lane's row of 16 (DPP row_newbcast: no LDS round trip per unit).
template <int HH>
__device__ __forceinline__ void ild_w2_terms(float& sc, float acc, const float* w2, int H) {
  if constexpr (HH < 16) {
    if (HH < H) {
      const float ah = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc), 0x150 + HH, 0xF, 0xF, false));
      sc = sc + w2[HH] * fmaxf(ah, 0.f);
    }
    ild_w2_terms<HH + 1>(sc, acc, w2, H);
  }
}

// float -> uint32 preserving order (so 64-bit keys (score, ~token) compare by score desc, token asc)
__device__ __forceinline__ uint32_t ild_fkey(float s) {
  const uint32_t u = __float_as_uint(s + 0.0f);
  return (u >> 31) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float ild_logf(float x) { return (float)log((double)x); }
__device__ __forceinline__ float ild_expf(float x) { return (float)exp((double)x); }

// The next pass's rows, tree and control block from the drafted rows (one thread).
__device__ __forceinline__ void ild_next_pass(const IllPassArgs& a, const IldLds& S, int treeB) {
  IllCtl* c = a.ctl;
  int rows;
  if (treeB > 0) {
    rows = S.rows;
    a.tree[0] = rows;
    for (int i = 0; i < rows; ++i) {
      a.tree[ILL_TR_DEPTH + i] = S.tr_dep[i];
      a.tree[ILL_TR_PARENT + i] = i == 0 ? -1 : S.tr_par[i];
      a.tree[ILL_TR_TOK + i] = S.tr_tok[i];
      a.tree[ILL_TR_ANC + i] = (int)S.tr_anc[i];
      a.ptoks[i] = S.tr_tok[i];
    }
    c->mode = ILL_MODE_TREE;
  } else {
    rows = 1 + S.nd;
    for (int i = 0; i < rows; ++i) a.ptoks[i] = S.next_rows[i];
    c->mode = ILL_MODE_ROWS;
  }
  a.st->n = rows;
  a.st->nver = rows;
  a.st->tree = treeB > 0 ? 1 : 0;
  c->nrows = rows;
  c->lmh_row0 = 0;
  c->lmh_rows = rows;
  c->commit = 2;
  c->draft = 0;
}

__global__ __launch_bounds__(ILD_THREADS) void ill_ildraft_kernel(IllPassArgs a, IllDraftArgs d) {
  __shared__ IldLds S;
  __shared__ int go0, have, w0, base, T, K, treeB, first_out, last, eos0, eos1;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  if (tid == 0) {
    const IllState* st = a.st;
    go0 = a.ctl->draft && !st->done;
    have = st->step;
    w0 = have > ILL_OB_MAX ? have - ILL_OB_MAX : 0;
    base = have - w0;
    T = min(max(st->tspec, 1), ILL_MAXT);
    treeB = a.ctl->tree_b;
    K = st->nodraft ? 0 : (treeB > 0 ? min(treeB, T - 1) : T - 1);
    eos0 = st->eos0;
    eos1 = st->eos1;
    go0 = go0 && have >= 1;
    first_out = go0 ? a.out_dev[0] : 0;
    last = go0 ? a.out_dev[have - 1] : 0;
    S.ticks0 = 0;
  }
  __syncthreads();
  if (!go0) return;
  if (K == 0) {   // nothing to draft: the next pass is the one row `last` (nothing to stage)
    if (tid == 0) {
      S.rows = 1;
      S.nd = 0;
      S.tr_par[0] = -1;
      S.tr_tok[0] = last;
      S.tr_dep[0] = 0;
      S.tr_anc[0] = 1u;
      S.next_rows[0] = last;
      ild_next_pass(a, S, treeB);
    }
    return;
  }
  // stage the request and the scorer
  {
    const int4* src = (const int4*)d.req;
    int4* dst = (int4*)&S.R;
    for (int k = tid; k < (int)(sizeof(IllDraftReq) / 16); k += ILD_THREADS) dst[k] = src[k];
    const float* m = (const float*)(d.tab + d.mlp);
    const int H = d.H;
    for (int k = tid; k < H * ILD_W1S; k += ILD_THREADS) {
      const int h = k / ILD_W1S, i = k - h * ILD_W1S;
      S.w1[k] = i < ILD_NF ? m[h * ILD_NF + i] : 0.f;
    }
    if (tid < H) {
      S.b1[tid] = m[H * ILD_NF + tid];
      S.w2[tid] = m[H * ILD_NF + H + tid];
    }
    if (tid < ILD_W1S) S.wl[tid] = tid < ILD_NF ? m[H * ILD_NF + 2 * H + 1 + tid] : 0.f;
    if (tid == 0) S.b2 = m[H * ILD_NF + 2 * H];
    if (tid < ILD_LG1P) S.lg1p[tid] = ild_logf(1.f + (float)tid);
  }
  for (int k = tid; k < base; k += ILD_THREADS) S.ob[k] = a.out_dev[w0 + k];
  {
    int tk = 0;
    for (int k = tid; k < have; k += ILD_THREADS) {
      const int t = a.out_dev[k];
      tk += (t >= 0 && t < ILD_VOCAB) ? (d.tflg[t] & 7) : 0;
    }
    if (tk) atomicAdd(&S.ticks0, tk);
  }
  __syncthreads();
  if (tid == 0) {
    S.ticks = S.ticks0;
    S.depth = 0;
    S.nd = 0;
    S.go = K > 0 ? 1 : 0;
    S.rows = 1;
    S.erow = 0;
    S.h_n = 0;
    S.h_ctr = 0;
    S.tr_par[0] = -1;
    S.tr_tok[0] = last;
    S.tr_dep[0] = 0;
    S.tr_anc[0] = 1u;
    S.tr_cum[0] = 1.f;
    S.tr_tf[0] = 0;
    S.next_rows[0] = last;
  }
  const int MAXM = d.MAXM;
  const int vocab = a.W.vocab;
  for (int it = 0; it < 64; ++it) {
    __syncthreads();
    if (!S.go) break;
    const int Lo = base + S.depth, Lfull = have + S.depth, L = 5 + Lo;
    const int ticks = S.ticks;
    auto ctx = [&](int i) { return i < 5 ? ild_tail(i) : S.ob[i - 5]; };
    // ---- phase 0: the window's token set; clear the candidate set ----
    S.used[tid] = -1;
    S.cset[tid] = -1;
    if (tid == 0) S.nu = 0;
    __syncthreads();
    if (tid < Lo) ild_insert(S.used, S.ob[tid]);
    __syncthreads();
    // ---- phase A: sources ----
    if (w == 0) {
      // n-gram table: order n = g + 1 in lane group g (10 lanes each)
      const int g = lane / 10, gl = lane - g * 10, n = g + 1;
      const bool act = g < 6 && n <= d.N && n <= L;
      uint64_t key = 0;
      if (act) {
        uint64_t h = 0xcbf29ce484222325ull;
        h ^= (uint64_t)n;
        h *= 0x100000001b3ull;
        for (int i = L - n; i < L; ++i) {
          const uint32_t t = (uint32_t)ctx(i);
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            h ^= (uint64_t)((t >> (8 * b)) & 0xffu);
            h *= 0x100000001b3ull;
          }
        }
        key = h;
      }
      uint32_t vx = 0, vy = 0;
      const bool hit = act && ild_hfind(d.hng, d.bng, key, vx, vy);   // NGVL's entry of the key
      int tot = -1, cnt = 0, etok = 0, ecnt = 0;
      if (hit) {
        tot = (int)vx;
        cnt = (int)(vy & 7);
        if (gl < cnt) {
          const uint2 e = *(const uint2*)(d.tab + d.ngnx + (size_t)((vy >> 3) + gl) * 8);
          etok = (int)e.x;
          ecnt = (int)e.y;
          S.top_tok[n][gl] = etok;
          S.top_cnt[n][gl] = ecnt;
        }
      }
      if (g < 6 && gl == 0) {
        S.dist_tot[n] = tot;
        S.dist_cnt[n] = cnt;
      }
      // summary over the orders (every lane computes it from shuffles)
      int ln = 0, s3 = 0, s10 = 0, lcnt = 0, ltot = 0;
#pragma unroll
      for (int o = 1; o <= 6; ++o) {
        const int to = __shfl(tot, (o - 1) * 10, 64);
        const int co = __shfl(cnt, (o - 1) * 10, 64);
        if (to >= 0) {
          ln = o;
          lcnt = co;
          ltot = to;
          if (to >= 3) s3 = o;
          if (to >= 10) s10 = o;
        }
      }
      int toplong = -1, entlow = 0;
      if (ln > 0) {
        toplong = __shfl(etok, (ln - 1) * 10, 64);
        // entropy of the longest order's continuations: the terms pr * ln(pr) in parallel
        // (lane r of that order's group), summed in order r = 0, 1, ...
        float term = 0.f;
        if (g == ln - 1 && gl < lcnt) {
          const float pr = (float)ecnt / (float)ltot;
          term = pr * ild_logf(pr);
        }
        float ent = 0.f;
        for (int r = 0; r < lcnt; ++r) ent = ent - __shfl(term, (ln - 1) * 10 + r, 64);
        entlow = ent < 0.3f ? 1 : 0;
      }
      if (lane == 0) {
        S.s_long = ln;
        S.s_supp3 = s3;
        S.s_supp10 = s10;
        S.s_toplong = toplong;
        S.s_entlow = entlow;
      }
    } else if (w == 1) {
      // self-repetition: the longest suffix (<= MAXM) of the window seen earlier, latest
      uint32_t best = 0;
      for (int e = lane + 1; e <= Lo - 1; e += 64) {
        const int lim = min(min(MAXM, Lo - 1), e);
        int m = 0;
        while (m < lim && S.ob[e - 1 - m] == S.ob[Lo - 1 - m]) m++;
        if (m > 0) {
          const uint32_t k = ((uint32_t)m << 16) | (uint32_t)e;
          best = k > best ? k : best;
        }
      }
      best = ild_wave_max(best);
      if (lane == 0) {
        S.self_n = (int)(best >> 16);
        S.self_tok = best ? S.ob[best & 0xffff] : -1;
      }
    } else if (w == 2) {
      // prompt lookup: every occurrence (ascending, first 32) of the longest suffix in P
      const int np = S.R.np;
      uint32_t mx = 0;
      for (int e = lane + 1; e <= np - 1; e += 64) {
        const int lim = min(min(MAXM, Lo), e);
        int m = 0;
        while (m < lim && S.R.P[e - 1 - m] == S.ob[Lo - 1 - m]) m++;
        S.pm[e] = m;
        mx = (uint32_t)m > mx ? (uint32_t)m : mx;
      }
      mx = ild_wave_max(mx);
      ild_wave_sync();
      int cnt = 0;
      if (mx > 0) {
        for (int e0 = 1; e0 <= np - 1 && cnt < 32; e0 += 64) {
          const int e = e0 + lane;
          const bool pred = e <= np - 1 && S.pm[e] == (int)mx;
          const uint64_t bal = __ballot(pred);
          const int pos = cnt + __popcll(bal & ((1ull << lane) - 1));
          if (pred && pos < 32) S.pr_tok[pos] = S.R.P[e];
          cnt += __popcll(bal);
        }
      }
      if (lane == 0) {
        S.pr_n = (int)mx;
        S.pr_cnt = min(cnt, 32);
      }
    } else if (w == 3) {
      // copy context: rates after the last token (CPC1) and the last two (CPC2)
      const uint32_t c_1 = (uint32_t)ctx(L - 1), c_2 = (uint32_t)ctx(L - 2);
      uint32_t rate = 0, unused = 0;
      if (lane == 0) S.c1 = ild_hfind(d.hc1, d.bc1, (uint64_t)c_1, rate, unused) ? __uint_as_float(rate) : 0.1f;
      if (lane == 32) S.c2 = ild_hfind(d.hc2, d.bc2, ((uint64_t)c_2 << 32) | c_1, rate, unused) ? __uint_as_float(rate) : 0.1f;
      // the first prompt token not in the window whose copy rate exceeds 0.3
      uint32_t fu = 0xffffffffu;
      for (int i = lane; i < S.R.np; i += 64)
        if (!ild_has(S.used, S.R.P[i]) && S.R.pprop[i] > 0.3f) fu = min(fu, (uint32_t)i);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) fu = min(fu, (uint32_t)__shfl_xor((int)fu, off, 64));
      if (lane == 0) S.firstun = fu != 0xffffffffu ? S.R.P[fu] : -1;
    } else if (w < 4 + ILD_MAXNB / 2) {
      // neighbour k: the longest suffix (<= MAXM) of TAIL + window in its sequence, first occurrence
      const int k = (w - 4) * 2 + (lane >> 5), sl = lane & 31;
      uint64_t key = 0;
      int a0 = 0;
      if (k < S.R.nnb) {
        a0 = S.R.nbOff[k];
        const int ls = S.R.nbOff[k + 1] - a0;
        for (int e = sl + 1; e <= ls - 1; e += 32) {
          const int lim = min(min(MAXM, L), e);
          int m = 0;
          while (m < lim && S.R.nbTok[a0 + e - 1 - m] == ctx(L - 1 - m)) m++;
          if (m > 0) {
            const uint64_t kk = ((uint64_t)m << 16) | (uint64_t)(0xffff - e);
            key = kk > key ? kk : key;
          }
        }
      }
      key = ild_max64(key, 32);
      if (sl == 0) {
        if (k < S.R.nnb && key) {
          S.vote_tok[k] = S.R.nbTok[a0 + (0xffff - (int)(key & 0xffff))];
          S.vote_n[k] = (int)(key >> 16);
        } else {
          S.vote_tok[k] = -1;
          S.vote_n[k] = 0;
        }
      }
    }
    __syncthreads();
    // ---- phase B: the distinct candidates ----
    {
      const int nraw = 85 + S.R.ncopy;
      if (tid < nraw) {
        const int i = tid;
        int t;
        if (i < 36) {
          const int n = i / 6 + 1, r = i % 6;
          t = (S.dist_tot[n] >= 0 && r < S.dist_cnt[n]) ? S.top_tok[n][r] : -1;
        } else if (i == 36) {
          t = S.self_n > 0 ? S.self_tok : -1;
        } else if (i < 53) {
          t = S.vote_tok[i - 37];
        } else if (i < 85) {
          t = i - 53 < S.pr_cnt ? S.pr_tok[i - 53] : -1;
        } else {
          t = S.R.copyTok[i - 85];
        }
        if (t >= 0 && t < vocab && ild_insert(S.cset, t)) S.uniq[atomicAdd(&S.nu, 1)] = t;
      }
    }
    __syncthreads();
    const int nu = S.nu;
    // ---- phase C1: features into LDS rows, two threads per candidate: waves 0-7 the
    // n-gram, self-repetition, prompt and neighbour features (0-28, 31, 32), waves 8-15 the
    // copy, association and token features (29, 30, 33-52) ----
    if ((tid & 511) < nu) {
      const int c = tid & 511;
      const int tok = S.uniq[c];
      float* f = S.F + c * ILD_FS;
      if (tid < 512) {
        for (int i = 0; i < 29; ++i) f[i] = 0.f;
        f[0] = 1.f;
        float f2 = 0.f, f17 = 0.f, f25;
        const int ln = S.s_long;
        for (int n = 1; n <= 6; ++n) {
          const int tot = S.dist_tot[n];
          if (tot < 0) continue;
          const int cnt = S.dist_cnt[n];
          int cn = 0, rank = -1;
          for (int r = 0; r < cnt; ++r)
            if (S.top_tok[n][r] == tok) {
              cn = S.top_cnt[n][r];
              rank = r;
              break;
            }
          if (n == ln && rank == 1) f[13] = 1.f;
          if (n == ln && rank >= 2) f[14] = 1.f;
          if (cn > 0) {
            const float p = (float)cn / (float)tot;
            f[6 + n] = p;
            if (n == ln) {
              f[1] = p;
              f[3] = ((float)n / 6.f) * p;
              f[4] = cn < ILD_LG1P ? S.lg1p[cn] : ild_logf(1.f + (float)cn);
            }
            if (n == S.s_supp3) f[5] = p;
            if (n == S.s_supp10) f[6] = p;
          }
        }
        if (tok == S.s_toplong) {
          f[2] = f2 = 1.f;
          if (S.s_entlow) f[15] = 1.f;
        }
        const int sn = S.self_n;
        if (sn > 0 && tok == S.self_tok) {
          f[16] = (float)sn / 4.f;
          f[17] = f17 = 1.f;
          f[18] = sn >= 3 ? 1.f : 0.f;
        }
        for (int q = 0; q < S.pr_cnt; ++q)
          if (S.pr_tok[q] == tok) {
            f[19] = (float)S.pr_n / 4.f;
            f[20] = 1.f;
            f[21] = S.pr_n >= 2 ? 1.f : 0.f;
            if (q == 0) f[22] = 1.f;
          }
        {
          const int nnb = S.R.nnb;
          float nbs = 0.f, nbm = 0.f, nbx = 0.f;
          int nbc = 0;
          for (int k = 0; k < nnb; ++k) {
            if (S.vote_tok[k] != tok) continue;
            const float sk = S.R.nbScore[k], mk = (float)min(S.vote_n[k], 8) / 8.f;
            nbs = nbs + sk;
            nbm = nbm + sk * mk;
            nbc++;
            nbx = fmaxf(nbx, mk);
            if (k == 0) {
              f[27] = 1.f;
              f[28] = mk;
            }
          }
          f[23] = nbs;
          f[24] = nbm;
          f[25] = f25 = (float)nbc / (float)max(1, nnb);
          f[26] = nbx;
        }
        f[31] = f2 * fminf(1.f, 2.f * f25);
        f[32] = f17 * fminf(1.f, 2.f * f25);
      } else {
        f[29] = 0.f;
        f[30] = 0.f;
        for (int i = 33; i < ILD_NF; ++i) f[i] = 0.f;
        const int ci = ild_bsearch(S.R.copyTok, S.R.ncopy, tok);
        const bool usedt = ild_has(S.used, tok);
        const bool inp = ci >= 0 && S.R.copyInP[ci] != 0;
        if (ci >= 0) {
          f[33] = S.R.copyF33[ci];
          f[34] = S.c1;
          f[35] = S.c2;
          f[36] = usedt ? 0.f : 1.f;
          f[37] = tok == S.firstun ? 1.f : 0.f;
          f[38] = inp ? 0.f : 1.f;
        }
        f[29] = (tok == 151645 || tok == 151643) ? 1.f : 0.f;
        f[30] = inp ? 1.f : 0.f;
        f[39] = (Lfull > 0 && (first_out == 73594 || first_out == 13874)) ? 1.f : 0.f;
        f[40] = (Lfull > 0 && first_out == 63) ? 1.f : 0.f;
        const uint32_t tf = tok < ILD_VOCAB ? (uint32_t)d.tflg[tok] : 0u;
        f[41] = (tf & 7u) ? 1.f : 0.f;
        f[42] = (tf & 8u) ? 1.f : 0.f;
        f[43] = (float)(ticks & 1);
        f[44] = (float)min(Lfull, 32) / 32.f;
        f[45] = usedt ? 1.f : 0.f;
        const int ai = ild_bsearch(S.R.asTok, S.R.nas, tok);
        if (ai >= 0) {
          f[46] = S.R.asMax[ai] / 4.f;
          f[47] = (float)min(S.R.asCnt[ai], 4) / 4.f;
        }
        S.ctf[c] = (int)(tf & 7u);
      }
    }
    __syncthreads();
    // ---- phase C2: the scorer, HL lanes per candidate (lane h: hidden unit h) ----
    //   a_h = b1[h] + W1[h][0] f[0] + ... + W1[h][52] f[52]        (left to right)
    //   sc  = b2 + WL[0] f[0] + ... + WL[52] f[52] + W2[0] relu(a_0) + ... + W2[H-1] relu(a_{H-1})
    // every product and sum rounded to float32 (no contraction), the order of a one-thread loop
    uint64_t mykey = 0;
    {
      const int H = d.H;
      const int HL = H <= 16 ? 16 : 32;
      const int h = tid & (HL - 1), gbase = lane & ~(HL - 1);
      for (int c0 = 0; c0 < nu; c0 += ILD_THREADS / HL) {
        const int c = c0 + tid / HL;
        const float4* fr = (const float4*)(S.F + min(c, nu - 1) * ILD_FS);
        const float4* wl = (const float4*)S.wl;
        // the hidden unit's chain and the linear term's chain advance together (two
        // independent dependency chains in one loop; each keeps its own order); the feature
        // row and the linear weights are read four at a time
        const float* wr = S.w1 + min(h, H - 1) * ILD_W1S;
        float acc = S.b1[min(h, H - 1)];
        float sc = S.b2;
#pragma unroll 2
        for (int i4 = 0; i4 < ILD_FS / 4; ++i4) {
          const float4 x4 = fr[i4], l4 = wl[i4];
          const float xs[4] = {x4.x, x4.y, x4.z, x4.w}, ls[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int i = 4 * i4 + q;
            if (i < ILD_NF) {
              acc = acc + wr[i] * xs[q];
              sc = sc + ls[q] * xs[q];
            }
          }
        }
        if (h >= H) acc = 0.f;
        if (HL == 16) {   // a candidate's 16 lanes are a DPP row: row_newbcast hands lane hh's unit to all
          ild_w2_terms<0>(sc, acc, S.w2, H);
        } else {
          for (int hh = 0; hh < H; ++hh) {
            const float ah = __shfl(acc, gbase + hh, 64);
            sc = sc + S.w2[hh] * fmaxf(ah, 0.f);
          }
        }
        if (h == 0 && c < nu) {
          const uint64_t key = ((uint64_t)ild_fkey(sc) << 32) | (uint64_t)(0xffffffffu - (uint32_t)S.uniq[c]);
          S.csc[c] = sc;
          S.ckey[c] = key;
          mykey = key > mykey ? key : mykey;
        }
      }
    }
    // ---- phase D: the best candidate; for trees the top 8 and the normaliser ----
    {
      const uint64_t m = ild_max64(mykey, 64);
      if (lane == 0) S.red64[w] = m;
      __syncthreads();
      uint64_t best = 0;
#pragma unroll
      for (int k = 0; k < ILD_THREADS / 64; ++k) best = S.red64[k] > best ? S.red64[k] : best;
      if (treeB > 0) {
        // the best score is the one whose key is `best` (every thread can rebuild it)
        const uint32_t fk = (uint32_t)(best >> 32);
        const float bs = __uint_as_float((fk & 0x80000000u) ? (fk & 0x7fffffffu) : ~fk);
        const float mx = fmaxf(nu > 0 ? bs : 0.f, 0.f);
        double ez = 0.0;
        if (tid < nu) {
          const uint64_t key = S.ckey[tid];
          const float e = ild_expf(S.csc[tid] - mx);
          ez = (double)e;
          int rank = 0;
          for (int j = 0; j < nu; ++j) rank += S.ckey[j] > key ? 1 : 0;
          if (rank < 8) {
            S.tk_tok[rank] = S.uniq[tid];
            S.tk_e[rank] = e;
            S.tk_tf[rank] = S.ctf[tid];
          }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ez += __shfl_xor(ez, off, 64);
        if (lane == 0) S.redd[w] = ez;
        __syncthreads();
        if (w == 0) {
          // push the expanded row's top children, then pop best-first (cumulative
          // probability desc, insertion order asc) until a row to expand or a full tree
          double z = (double)ild_expf(-mx);
          for (int k = 0; k < ILD_THREADS / 64; ++k) z += S.redd[k];
          const float Z = (float)z;
          const int hn0 = S.h_n, ctr0 = S.h_ctr, erow0 = S.erow;
          const int npush = min(min(8, nu), ILD_HEAP - hn0);
          const float pc = S.tr_cum[erow0];
          if (lane < npush) {
            const int q = hn0 + lane;
            S.h_cum[q] = (pc * S.tk_e[lane]) / Z;
            S.h_par[q] = erow0;
            S.h_tok[q] = S.tk_tok[lane];
            S.h_tf[q] = S.tk_tf[lane];
            S.h_ord[q] = ctr0 + lane;
          }
          ild_wave_sync();
          if (lane == 0) {
            S.h_n = hn0 + npush;
            S.h_ctr = ctr0 + npush;
          }
          ild_wave_sync();
          int go = 0;
          for (int pop = 0; pop < ILD_HEAP; ++pop) {
            const int hn = S.h_n;
            if (!(S.rows < K + 1 && hn > 0)) break;
            uint64_t kk = 0;
            for (int q = lane; q < hn; q += 64) {
              const uint64_t kq = ((uint64_t)__float_as_uint(S.h_cum[q]) << 32) |
                                  ((uint64_t)(0xffff - S.h_ord[q]) << 16) | (uint64_t)q;
              kk = kq > kk ? kq : kk;
            }
            kk = ild_max64(kk, 64);
            if (lane == 0) {
              const int b = (int)(kk & 0xffff);
              const float cum = S.h_cum[b];
              const int par = S.h_par[b], tkn = S.h_tok[b], tkf = S.h_tf[b];
              const int hl = hn - 1;
              S.h_cum[b] = S.h_cum[hl];
              S.h_par[b] = S.h_par[hl];
              S.h_tok[b] = S.h_tok[hl];
              S.h_tf[b] = S.h_tf[hl];
              S.h_ord[b] = S.h_ord[hl];
              S.h_n = hl;
              const int i = S.rows;
              S.rows = i + 1;
              S.tr_par[i] = par;
              S.tr_tok[i] = tkn;
              S.tr_tf[i] = tkf;
              S.tr_dep[i] = S.tr_dep[par] + 1;
              S.tr_anc[i] = S.tr_anc[par] | (1u << i);
              S.tr_cum[i] = cum;
              const int expand = !(tkn == eos0 || tkn == eos1 || i + 1 == K + 1);
              if (expand) {
                S.depth = S.tr_dep[i];
                S.erow = i;
              }
              S.flag = expand;
            }
            ild_wave_sync();
            if (S.flag) {
              // the expanded row's path into the window: its rows j > 0 are the set bits of
              // tr_anc (one lane each), row j's token at depth tr_dep[j]; the ticks add theirs
              const uint32_t anc = S.tr_anc[S.erow];
              int tf = 0;
              if (lane > 0 && lane < 32 && ((anc >> lane) & 1u)) {
                S.ob[base + S.tr_dep[lane] - 1] = S.tr_tok[lane];
                tf = S.tr_tf[lane];
              }
              tf = gsumi<64>(tf);
              if (lane == 0) S.ticks = S.ticks0 + tf;
              go = 1;
              break;
            }
          }
          if (lane == 0) S.go = go;
        }
      } else {
        if (tid < nu && S.ckey[tid] == best) S.best_tf = S.ctf[tid];
        __syncthreads();
        if (tid == 0) {
          if (nu == 0) {
            S.go = 0;
          } else {
            const int bt = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
            const int nd = S.nd;
            S.next_rows[nd + 1] = bt;
            S.ob[Lo] = bt;
            S.nd = nd + 1;
            S.depth = nd + 1;
            S.ticks = ticks + S.best_tf;
            S.go = (nd + 1 < K && bt != eos0 && bt != eos1) ? 1 : 0;
          }
        }
      }
    }
  }
  __syncthreads();
  if (tid == 0) ild_next_pass(a, S, treeB);
}
