// The pass kernel: one persistent launch runs a whole decode step, prefill chunk or
// tree-verify pass over T rows (T = 1 or 16 at compile time; `nrows` <= T at run time).
//
// The reference encodes the same work as 24 x 5 + 2 dependent dispatches
// (Sources/Engine/Engine.swift:245-292, :605-609). Here 256 workgroups stay resident and
// each takes one role per layer; roles hand data to each other through tagged words
// (ill_device.h), so a consumer waits only for the words it needs:
//
//   QKV  (36 WGs)  x_l -> RMSNorm -> 32-row rotary block of QKV -> bias, RoPE, q / K / V
//   ATT  (28 WGs)  (kv group, row): MFMA flash attention over 64-position chunks
//   O    (56 WGs)  attention output -> 16-row tile of O -> + residual -> x'
//   GUD  (76 WGs)  x' -> RMSNorm -> 64 hidden units of gate/up -> SiLU*up -> down partial
//   RED  (56 WGs)  x' + sum of the 76 down partials (fixed order) -> x_{l+1}
//   LMH  (all)     final RMSNorm -> tied lm_head tiles -> per-WG argmax partials
//   COMMIT (WG 0)  argmax (ties -> lowest id), token record, state advance, tree accept,
//                  KV compaction, epoch advance
//
// Every role issues its weight loads for a layer before it waits for that layer's input,
// so HBM streaming overlaps the dependency chain.
#pragma once
#include "ill_device.h"

struct IllPassArgs {
  IllWeights W;
  const IllLayerW* L;
  IllState* st;
  IllCtl* ctl;
  int32_t* ptoks;          // [16] row tokens of the pass (commit writes [0] for the next step)
  const int32_t* tree;     // [65]
  const float2* rope;      // [maxctx + 16][32] (cos, sin)
  uint16_t* kc;            // K cache [layer][kvh][maxctx][64] f16
  uint16_t* vt;            // V cache transposed per 64 slots [layer][kvh][maxctx/64][64 dims][64] f16
  uint64_t* xa;            // [16][896] layer input
  uint64_t* xb;            // [16][896] residual after attention
  uint64_t* q;             // [16][896] rotated queries
  uint64_t* kvn;           // [16][kvh 2][k/v 2][32] this pass's K/V rows: word d = f16 pair (d, d+32)
  uint64_t* attn;          // [16][896]
  uint64_t* part;          // [76][16][896] down partials
  uint64_t* lmp;           // [256][16][2] lm_head argmax partials (value, index)
  float* logits;           // [16][V]
  int32_t* out_dev;        // [maxsteps]
  int32_t* out_host;       // [maxsteps] pinned host memory
  uint64_t* trace;         // optional [256][ILL_TRACE_SLOTS] timestamps (nullptr = off)
  int maxctx;
  int maxsteps;
};

// Trace slots per workgroup: 3 per layer (role start, input ready, output written) and
// 3 for the lm_head / commit tail.
#define ILL_TRACE_SLOTS (3 * ILL_MAXLAYERS + 6)
__device__ __forceinline__ void trace_mark(const IllPassArgs& a, int slot) {
  if (a.trace && threadIdx.x == 0) a.trace[blockIdx.x * ILL_TRACE_SLOTS + slot] = wall_clock64();
}

struct PassHdr {
  uint32_t epoch;
  int mode, nrows, pos, lmh0, lmhn, wlog, commit, done;
  int tok[16], depth[16], parent[16];
};

struct AttLds {
  v8h qa[2 * 2 * 64];            // [ks][hi/lo][lane]
  float P[ILL_WAVES][8][64];     // per-wave softmax weights of one chunk
  float cm[ILL_WAVES][8], cl[ILL_WAVES][8];
  float co[ILL_WAVES][7][64];
  int prow[16];
};

struct GudLds {
  PrepLds prep;
  float gu[8][16][16];           // [tile][row][unit]
  uint4 ahi[4 * 16], alo[4 * 16];
  float2 dsc[16];
};

struct LmhLds {
  PrepLds prep;
  float bv[ILL_WAVES][16];
  int bi[ILL_WAVES][16];
};

struct CommitLds {
  float v[256];
  int i[256];
  int g[16];
  int path[16];
  int npath, pos0;
};

union PassLds {
  PrepLds prep;
  AttLds att;
  GudLds gud;
  LmhLds lmh;
  CommitLds cm;
};

__device__ __forceinline__ uint32_t tagof(uint32_t epoch, int layer) { return epoch * 32u + (uint32_t)layer + 1u; }

// ---- activation sources for prep896 --------------------------------------------------
struct SrcTagged {
  const uint64_t* base;
  uint32_t tag;
  __device__ __forceinline__ bool load(int t, int c0, float* v) const {
    const uint64_t* p = base + t * ILL_H + c0;
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint64_t w = aload64(p + i);
      ok &= wok(w, tag);
      v[i] = wval(w);
    }
    return ok;
  }
};

// Embedding rows (layer-0 input), dequantized from the tiled q4 table: w = s*q + m
// (Shaders.swift:118-126 semantics).
__device__ __forceinline__ void embed16(const IllWeights& W, int tok, int c0, float* v) {
  const int rt = tok >> 4, n = tok & 15;
  const int cb = c0 >> 7, gi = (c0 >> 6) & 1, kg = (c0 >> 4) & 3;
  const uint8_t* blk = W.wemb + ((size_t)rt * ILL_KST + cb) * 1024 + (kg * 16 + n) * 16 + gi * 8;
  const uint2 b = *(const uint2*)blk;
  const uint32_t sm = W.semb[((size_t)rt * ILL_KST + cb) * 32 + n * 2 + gi];
  const float s = h2f(sm & 0xffff), m = h2f(sm >> 16);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t word = i < 8 ? b.x : b.y;
    const int k = i & 7;
    const uint32_t q = (word >> (4 * k)) & 0xF;
    v[i] = s * (float)q + m;
  }
}

__device__ __forceinline__ float embed1(const IllWeights& W, int tok, int c) {
  float v[16];
  embed16(W, tok, c & ~15, v);
  return v[c & 15];
}

struct SrcEmbed {
  IllWeights W;
  const int* toks;   // LDS copy of the row tokens
  __device__ __forceinline__ bool load(int t, int c0, float* v) const {
    embed16(W, toks[t], c0, v);
    return true;
  }
};

// RMSNorm (optional) + 16-bit fixed-point coding of rows 0..nrows-1 of a K = 896 input
// into MFMA operands. Row t is handled by wave t % 8 with the same instruction sequence
// for every T: lane (G, kg) = (lane / 4, lane % 4), lanes 56-63 idle.
template <int T, class Src>
__device__ __forceinline__ bool prep896(const Src& src, const float* gamma, int nrows, PrepLds& P,
                                        IllCtl* ctl, int code) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = lane >> 2, kg = lane & 3;
  const bool act = lane < 56;
  const int c0 = 64 * G + 16 * kg;
  bool alive = true;
  for (int t = w; t < T && alive; t += ILL_WAVES) {
    if (t >= nrows) {
      if (act) {
        P.ahi[(G * 4 + kg) * 16 + t] = make_uint4(0, 0, 0, 0);
        P.alo[(G * 4 + kg) * 16 + t] = make_uint4(0, 0, 0, 0);
        if (kg == 0) P.sc[G * 16 + t] = make_float2(0.f, 0.f);
      }
      continue;
    }
    float v[16];
    alive = wave_wait([&]() { return !act || src.load(t, c0, v); }, ctl, code);
    if (!alive) break;
    if (!act) {
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = 0.f;
    }
    if (gamma) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i++) ss = fmaf(v[i], v[i], ss);
      ss = wsum64(ss);
      const float scale = 1.0f / sqrtf(ss / (float)ILL_H + ILL_EPS);
      if (act) {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = v[i] * scale * gamma[c0 + i];
      }
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = wmax_xor(mx, 1, 2);
    const float d = mx / ILL_QMAX;
    uint32_t hi[4], lo[4];
    int sq;
    quant16(v, d, hi, lo, sq);
    sq = isum_xor(sq, 1, 2);
    if (act) {
      P.ahi[(G * 4 + kg) * 16 + t] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
      P.alo[(G * 4 + kg) * 16 + t] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
      if (kg == 0) P.sc[G * 16 + t] = make_float2(d, d * (float)sq);
    }
  }
  __syncthreads();
  return !wg_failed(ctl);
}

// ---------------------------------------------------------------------------------------
template <int T>
__device__ bool role_qkv(const IllPassArgs& a, const PassHdr& H, PassLds& S, int l, int b) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const IllLayerW& L = a.L[l];
  Q4Tile t0, t1;
  if (w == 0) {
    q4_load(t0, L.wqkv + (size_t)(2 * b) * ILL_KST * 1024, L.sqkv + (2 * b) * ILL_KST * 32, lane);
    q4_load(t1, L.wqkv + (size_t)(2 * b + 1) * ILL_KST * 1024, L.sqkv + (2 * b + 1) * ILL_KST * 32, lane);
  }
  bool ok;
  if (l == 0) ok = prep896<T>(SrcEmbed{a.W, H.tok}, L.ln1, H.nrows, S.prep, a.ctl, 100 + l);
  else ok = prep896<T>(SrcTagged{a.xa, tagof(H.epoch, l)}, L.ln1, H.nrows, S.prep, a.ctl, 100 + l);
  if (!ok) return false;
  trace_mark(a, 3 * l + 1);
  if (w == 0) {
    float acc0[4] = {0.f, 0.f, 0.f, 0.f}, acc1[4] = {0.f, 0.f, 0.f, 0.f};
    q4_tile896<T>(t0, S.prep, lane, acc0);
    q4_tile896<T>(t1, S.prep, lane, acc1);
    const int kg = lane >> 4, n = lane & 15;
    const int head = b >> 1, d = (b & 1) * 16 + n;
    const float bias0 = L.bqkv[32 * b + n], bias1 = L.bqkv[32 * b + 16 + n];
    const uint32_t tag = tagof(H.epoch, l);
    constexpr int RPL = T >= 4 ? 4 : T;
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t >= H.nrows) continue;
      float x0 = acc0[j] + bias0, x1 = acc1[j] + bias1;
      const int slot = H.pos + t;
      if (head < ILL_NH + ILL_NKV) {
        const float2 cs = a.rope[(H.pos + H.depth[t]) * 32 + d];
        const float r0 = x0 * cs.x - x1 * cs.y;
        const float r1 = x1 * cs.x + x0 * cs.y;
        x0 = r0;
        x1 = r1;
      }
      if (head < ILL_NH) {
        astore64(a.q + t * ILL_H + head * 64 + d, mkw(x0, tag));
        astore64(a.q + t * ILL_H + head * 64 + d + 32, mkw(x1, tag));
      } else {
        const int kv = head < ILL_NH + ILL_NKV ? 0 : 1;
        const int kh = head - ILL_NH - kv * ILL_NKV;
        const uint32_t h0 = f2h(x0), h1 = f2h(x1);
        if (kv == 0) {
          uint16_t* kr = a.kc + (((size_t)l * ILL_NKV + kh) * a.maxctx + slot) * 64;
          kr[d] = (uint16_t)h0;
          kr[d + 32] = (uint16_t)h1;
        } else {
          uint16_t* vb = a.vt + (((size_t)l * ILL_NKV + kh) * (a.maxctx / 64) + slot / 64) * 64 * 64;
          vb[d * 64 + (slot & 63)] = (uint16_t)h0;
          vb[(d + 32) * 64 + (slot & 63)] = (uint16_t)h1;
        }
        astore64(a.kvn + ((t * 2 + kh) * 2 + kv) * 32 + d, mkwu(h0 | (h1 << 16), tag));
      }
    }
  }
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------------------------------
// Attention for one (kv group g, row t): virtual positions 0 .. L-1 with L = pos + depth + 1;
// position p < pos is cache slot p, p >= pos is pass row prow[p - pos] (this pass's K/V).
// Chunks of 64 positions go to wave (chunk % 8); each chunk is one MFMA flash-attention
// step; chunk results combine in chunk order per wave, then over waves 0..7. Nothing here
// depends on T, so a tree row and the same token decoded alone give identical bits.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ v8h u4_to_v8h(uint4 u) {
  v8h r;
  const uint32_t a[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t x = a[i];
    r[2 * i] = __builtin_bit_cast(_Float16, (unsigned short)(x & 0xffff));
    r[2 * i + 1] = __builtin_bit_cast(_Float16, (unsigned short)(x >> 16));
  }
  return r;
}

__device__ __forceinline__ _Float16 hbits(uint32_t b) { return __builtin_bit_cast(_Float16, (unsigned short)(b & 0xffff)); }

template <int T>
__device__ bool role_att(const IllPassArgs& a, const PassHdr& H, PassLds& S, int l, int g, int t) {
  AttLds& A = S.att;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int depth = H.depth[t];
  const int pos = H.pos;
  const int Lt = pos + depth + 1;
  const uint32_t tag = tagof(H.epoch, l);
  if (threadIdx.x == 0) {
    int r = t;
    for (int d = depth; d >= 0; --d) {
      A.prow[d] = r;
      r = r > 0 ? H.parent[r] : 0;
    }
  }
  __syncthreads();
  // wait for this row's queries and the K/V of every row on its path
  const int nkv = (depth + 1) * 64;
  const bool ok = wg_wait([&]() {
    bool r = true;
    const int i = threadIdx.x;
    if (i < 448) r &= wok(aload64(a.q + t * ILL_H + 7 * g * 64 + i), tag);
    for (int j = i; j < nkv; j += ILL_WG_THREADS) {
      const int row = A.prow[j >> 6], k = j & 63;
      r &= wok(aload64(a.kvn + ((row * 2 + g) * 2 + (k >> 5)) * 32 + (k & 31)), tag);
    }
    return r;
  }, a.ctl, 200 + l);
  if (!ok) return false;
  trace_mark(a, 3 * l + 1);
  // query operands: q * 0.125 split into f16 hi + lo; lane (kg, m = head), dims 32 ks + 8 kg + i
  {
    _Float16* qa = (_Float16*)A.qa;
    for (int i = threadIdx.x; i < 2 * 2 * 64 * 8; i += ILL_WG_THREADS) qa[i] = (_Float16)0.f;
    __syncthreads();
    if (threadIdx.x < 448) {
      const int h = threadIdx.x >> 6, dim = threadIdx.x & 63;
      const float v = wval(aload64(a.q + t * ILL_H + (7 * g + h) * 64 + dim)) * 0.125f;
      const _Float16 hi = (_Float16)v;
      const _Float16 lo = (_Float16)(v - (float)hi);
      const int ks = dim >> 5, kg = (dim >> 3) & 3, i = dim & 7;
      qa[((ks * 2 + 0) * 64 + kg * 16 + h) * 8 + i] = hi;
      qa[((ks * 2 + 1) * 64 + kg * 16 + h) * 8 + i] = lo;
    }
    __syncthreads();
  }
  const int kg = lane >> 4, n = lane & 15;
  const v8h qh0 = A.qa[(0 * 2 + 0) * 64 + lane], ql0 = A.qa[(0 * 2 + 1) * 64 + lane];
  const v8h qh1 = A.qa[(1 * 2 + 0) * 64 + lane], ql1 = A.qa[(1 * 2 + 1) * 64 + lane];
  const uint16_t* kbase = a.kc + ((size_t)l * ILL_NKV + g) * a.maxctx * 64;
  const uint16_t* vbase = a.vt + ((size_t)l * ILL_NKV + g) * (a.maxctx / 64) * 64 * 64;
  const uint64_t* kvk = a.kvn + (size_t)g * 2 * 32;   // + row * 128 words
  float M[4], Lw[4], O[4][4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    M[j] = -INFINITY;
    Lw[j] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; nb++) O[nb][j] = 0.f;
  }
  const int nch = (Lt + 63) >> 6;
  for (int c = w; c < nch; c += ILL_WAVES) {
    float sc[4][4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int vp = 64 * c + 16 * b + n;
      v8h k0, k1;
      if (vp < pos) {
        const uint4* kr = (const uint4*)(kbase + (size_t)vp * 64);
        k0 = u4_to_v8h(kr[kg]);
        k1 = u4_to_v8h(kr[4 + kg]);
      } else if (vp < Lt) {
        const uint64_t* kw = kvk + (size_t)A.prow[vp - pos] * 128 + 8 * kg;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const uint32_t x = (uint32_t)aload64(kw + i);
          k0[i] = hbits(x);
          k1[i] = hbits(x >> 16);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) { k0[i] = (_Float16)0.f; k1[i] = (_Float16)0.f; }
      }
      v4f s = {0.f, 0.f, 0.f, 0.f};
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh0, k0, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql0, k0, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh1, k1, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql1, k1, s, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; j++) sc[b][j] = vp < Lt ? s[j] : -INFINITY;
    }
    float mx[4], ls[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float m = fmaxf(fmaxf(sc[0][j], sc[1][j]), fmaxf(sc[2][j], sc[3][j]));
      mx[j] = wmax_xor(m, 1, 8);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float s = 0.f;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        sc[b][j] = expf(sc[b][j] - mx[j]);
        s += sc[b][j];
      }
      ls[j] = wsum_xor(s, 1, 8);
    }
    // P (heads < 8) to LDS, then PV operands: lane (kg, m = head), positions 32 ks + 8 kg + i
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int head = 4 * kg + j;
      if (head < 8) {
#pragma unroll
        for (int b = 0; b < 4; b++) A.P[w][head][16 * b + n] = sc[b][j];
      }
    }
    wave_lds_sync();
    v8h ph[2], pl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float p = n < 7 ? A.P[w][n][32 * ks + 8 * kg + i] : 0.f;
        const _Float16 hi = (_Float16)p;
        ph[ks][i] = hi;
        pl[ks][i] = (_Float16)(p - (float)hi);
      }
    }
    wave_lds_sync();
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
      const int dim = 16 * nb + n;
      v8h vv[2];
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const int p0 = 64 * c + 32 * ks + 8 * kg;
        if (p0 + 7 < pos) {
          const uint4 u = *(const uint4*)(vbase + ((size_t)c * 64 + dim) * 64 + 32 * ks + 8 * kg);
          vv[ks] = u4_to_v8h(u);
        } else {
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const int vp = p0 + i;
            uint32_t bits = 0;
            if (vp < pos) bits = vbase[((size_t)c * 64 + dim) * 64 + 32 * ks + 8 * kg + i];
            else if (vp < Lt) {
              const uint32_t x = (uint32_t)aload64(kvk + (size_t)A.prow[vp - pos] * 128 + 32 + (dim & 31));
              bits = dim < 32 ? (x & 0xffff) : (x >> 16);
            }
            vv[ks][i] = hbits(bits);
          }
        }
      }
      v4f o = {0.f, 0.f, 0.f, 0.f};
      o = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[0], vv[0], o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[0], vv[0], o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[1], vv[1], o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[1], vv[1], o, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float mn = fmaxf(M[j], mx[j]);
        const float sa = expf(M[j] - mn), sb = expf(mx[j] - mn);
        O[nb][j] = O[nb][j] * sa + o[j] * sb;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float mn = fmaxf(M[j], mx[j]);
      const float sa = expf(M[j] - mn), sb = expf(mx[j] - mn);
      Lw[j] = Lw[j] * sa + ls[j] * sb;
      M[j] = mn;
    }
  }
  // combine waves 0..7 in order
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int head = 4 * kg + j;
    if (head < 7) {
      if (n == 0) {
        A.cm[w][head] = M[j];
        A.cl[w][head] = Lw[j];
      }
#pragma unroll
      for (int nb = 0; nb < 4; nb++) A.co[w][head][16 * nb + n] = O[nb][j];
    }
  }
  __syncthreads();
  if (threadIdx.x < 448) {
    const int h = threadIdx.x >> 6, dim = threadIdx.x & 63;
    float m = -INFINITY, s = 0.f, o = 0.f;
    for (int ww = 0; ww < ILL_WAVES; ww++) {
      const float mw = A.cm[ww][h];
      if (mw == -INFINITY) continue;
      const float mn = fmaxf(m, mw);
      const float sa = expf(m - mn), sb = expf(mw - mn);
      s = s * sa + A.cl[ww][h] * sb;
      o = o * sa + A.co[ww][h][dim] * sb;
      m = mn;
    }
    astore64(a.attn + t * ILL_H + (7 * g + h) * 64 + dim, mkw(o / s, tag));
  }
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------------------------------
template <int T>
__device__ bool role_o(const IllPassArgs& a, const PassHdr& H, PassLds& S, int l, int ot) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const IllLayerW& L = a.L[l];
  Q4Tile tw;
  if (w == 0) q4_load(tw, L.wo + (size_t)ot * ILL_KST * 1024, L.so + ot * ILL_KST * 32, lane);
  const uint32_t tag = tagof(H.epoch, l);
  if (!prep896<T>(SrcTagged{a.attn, tag}, nullptr, H.nrows, S.prep, a.ctl, 300 + l)) return false;
  trace_mark(a, 3 * l + 1);
  bool alive = true;
  if (w == 0) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    q4_tile896<T>(tw, S.prep, lane, acc);
    const int kg = lane >> 4, n = lane & 15, row = 16 * ot + n;
    constexpr int RPL = T >= 4 ? 4 : T;
    float xin[4];
    alive = wave_wait([&]() {
      bool r = true;
#pragma unroll
      for (int j = 0; j < RPL; j++) {
        const int t = 4 * kg + j;
        if (t < H.nrows) {
          if (l == 0) xin[j] = embed1(a.W, H.tok[t], row);
          else {
            const uint64_t x = aload64(a.xa + t * ILL_H + row);
            r &= wok(x, tag);
            xin[j] = wval(x);
          }
        }
      }
      return r;
    }, a.ctl, 350 + l);
    if (alive) {
#pragma unroll
      for (int j = 0; j < RPL; j++) {
        const int t = 4 * kg + j;
        if (t < H.nrows) astore64(a.xb + t * ILL_H + row, mkw(xin[j] + acc[j], tag));
      }
    }
  }
  __syncthreads();
  return !wg_failed(a.ctl);
}

// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int q4perm_inv(int c) { return (c & 8) | ((c & 1) << 2) | ((c >> 1) & 3); }

template <int T>
__device__ bool role_gud(const IllPassArgs& a, const PassHdr& H, PassLds& S, int l, int ub) {
  GudLds& G = S.gud;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kg = lane >> 4, n = lane & 15;
  const IllLayerW& L = a.L[l];
  Q4Tile tg;
  q4_load(tg, L.wgu + (size_t)(ub * 8 + w) * ILL_KST * 1024, L.sgu + (ub * 8 + w) * ILL_KST * 32, lane);
  uint2 dw[7];
  uint32_t ds[7];
#pragma unroll
  for (int k = 0; k < 7; k++) {
    const int rt = 7 * w + k;
    dw[k] = *(const uint2*)(L.wd + ((size_t)ub * ILL_NOT + rt) * 512 + lane * 8);
    ds[k] = L.sd[(ub * ILL_NOT + rt) * 16 + n];
  }
  const uint32_t tag = tagof(H.epoch, l);
  if (!prep896<T>(SrcTagged{a.xb, tag}, L.ln2, H.nrows, G.prep, a.ctl, 400 + l)) return false;
  trace_mark(a, 3 * l + 1);
  constexpr int RPL = T >= 4 ? 4 : T;
  {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    q4_tile896<T>(tg, G.prep, lane, acc);
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t < T) G.gu[w][t][n] = acc[j];
    }
  }
  __syncthreads();
  // SiLU(gate) * up for the block's 64 units, then 16-bit coding of each row (group = 64)
  for (int t = w; t < T; t += ILL_WAVES) {
    if (t >= H.nrows) {
      if (lane < 4) {
        G.ahi[lane * 16 + t] = make_uint4(0, 0, 0, 0);
        G.alo[lane * 16 + t] = make_uint4(0, 0, 0, 0);
      }
      if (lane == 0) G.dsc[t] = make_float2(0.f, 0.f);
      continue;
    }
    const int u = lane, gi = u >> 4, nn = u & 15;
    const float gv = G.gu[gi][t][nn], up = G.gu[4 + gi][t][nn];
    const float h = gv / (1.0f + expf(-gv)) * up;
    const float mx = wmax_xor(fabsf(h), 1, 32);
    const float d = mx / ILL_QMAX;
    const int qv = d > 0.f ? (int)rintf(h / d) : 0;
    const int sq = isum_xor(qv, 1, 32);
    const int hi = (qv + 128) >> 8, lo = qv - (hi << 8);
    const int p = q4perm_inv(nn);
    uint8_t* bh = (uint8_t*)&G.ahi[gi * 16 + t];
    uint8_t* bl = (uint8_t*)&G.alo[gi * 16 + t];
    bh[p] = (uint8_t)(hi & 0xff);
    bl[p] = (uint8_t)(lo & 0xff);
    if (lane == 0) G.dsc[t] = make_float2(d, d * (float)sq);
  }
  __syncthreads();
  v4i ah = {0, 0, 0, 0}, al = {0, 0, 0, 0};
  if (n < T) {
    const uint4 x = G.ahi[kg * 16 + n], y = G.alo[kg * 16 + n];
    ah = (v4i){(int)x.x, (int)x.y, (int)x.z, (int)x.w};
    al = (v4i){(int)y.x, (int)y.y, (int)y.z, (int)y.w};
  }
  const v4i z = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < 7; k++) {
    const int rt = 7 * w + k;
    const v4i b = q4_unpack(dw[k].x, dw[k].y);
    const v4i dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, b, z, 0, 0, 0);
    const v4i dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, b, z, 0, 0, 0);
    const float sw = h2f(ds[k] & 0xffff), mw = h2f(ds[k] >> 16);
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t < H.nrows) {
        const float2 dx = G.dsc[t];
        const int Sv = (dh[j] << 8) + dl[j];
        float y = 0.f;
        y = fmaf(sw, dx.x * (float)Sv, y);
        y = fmaf(mw, dx.y, y);
        astore64(a.part + ((size_t)(ub * 16 + t)) * ILL_H + 16 * rt + n, mkw(y, tag));
      }
    }
  }
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------------------------------
template <int T>
__device__ bool role_red(const IllPassArgs& a, const PassHdr& H, int l, int rt) {
  const uint32_t tag = tagof(H.epoch, l);
  const int i = threadIdx.x;
  const int t = i >> 4, row = 16 * rt + (i & 15);
  const bool act = t < H.nrows;
  const bool ok = wg_wait([&]() {
    if (!act) return true;
    bool r = wok(aload64(a.xb + t * ILL_H + row), tag);
    for (int ub = 0; ub < ILL_NGU; ub++) r &= wok(aload64(a.part + ((size_t)(ub * 16 + t)) * ILL_H + row), tag);
    return r;
  }, a.ctl, 500 + l);
  if (!ok) return false;
  trace_mark(a, 3 * l + 1);
  if (act) {
    float acc = 0.f;
    for (int ub = 0; ub < ILL_NGU; ub++) acc += wval(aload64(a.part + ((size_t)(ub * 16 + t)) * ILL_H + row));
    const float x = wval(aload64(a.xb + t * ILL_H + row)) + acc;
    astore64(a.xa + t * ILL_H + row, mkw(x, tagof(H.epoch, l + 1)));
  }
  return true;
}

// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void amax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

template <int T>
__device__ bool role_lmh(const IllPassArgs& a, const PassHdr& H, PassLds& S) {
  LmhLds& Lm = S.lmh;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int NL = a.W.layers;
  const uint32_t tag = tagof(H.epoch, NL);
  const int V = a.W.vocab, ntiles = V >> 4;
  const int wg = blockIdx.x;
  float bv[4];
  int bi[4];
#pragma unroll
  for (int j = 0; j < 4; j++) { bv[j] = -INFINITY; bi[j] = 0x7fffffff; }
  if (H.lmhn > 0) {
    int tile = wg + ILL_WG * w;
    Q4Tile cur;
    if (tile < ntiles) q4_load(cur, a.W.wemb + (size_t)tile * ILL_KST * 1024, a.W.semb + (size_t)tile * ILL_KST * 32, lane);
    if (!prep896<T>(SrcTagged{a.xa, tag}, a.W.fnorm, H.nrows, Lm.prep, a.ctl, 600)) return false;
    trace_mark(a, 3 * ILL_MAXLAYERS + 1);
    constexpr int RPL = T >= 4 ? 4 : T;
    while (tile < ntiles) {
      const int nxt = tile + ILL_WG * ILL_WAVES;
      Q4Tile nx;
      if (nxt < ntiles) q4_load(nx, a.W.wemb + (size_t)nxt * ILL_KST * 1024, a.W.semb + (size_t)nxt * ILL_KST * 32, lane);
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      q4_tile896<T>(cur, Lm.prep, lane, acc);
      const int idx = 16 * tile + n;
#pragma unroll
      for (int j = 0; j < RPL; j++) {
        const int t = 4 * kg + j;
        if (t >= H.lmh0 && t < H.lmh0 + H.lmhn) {
          if (H.wlog) a.logits[(size_t)t * V + idx] = acc[j];
          amax_merge(bv[j], bi[j], acc[j], idx);
        }
      }
      cur = nx;
      tile = nxt;
    }
  }
  // per-row best over the 16 lanes of each lane-group, then over waves
#pragma unroll
  for (int j = 0; j < 4; j++) {
    for (int o = 8; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv[j], o, 64);
      const int oi = __shfl_xor(bi[j], o, 64);
      amax_merge(bv[j], bi[j], ov, oi);
    }
  }
  if (n == 0) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int t = 4 * kg + j;
      if (t < 16) { Lm.bv[w][t] = bv[j]; Lm.bi[w][t] = bi[j]; }
    }
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int t = threadIdx.x;
    float v = -INFINITY;
    int id = 0x7fffffff;
    if (t < T)
      for (int ww = 0; ww < ILL_WAVES; ww++) amax_merge(v, id, Lm.bv[ww][t], Lm.bi[ww][t]);
    astore64(a.lmp + (wg * 16 + t) * 2 + 0, mkw(v, tag));
    astore64(a.lmp + (wg * 16 + t) * 2 + 1, mkwu((uint32_t)id, tag));
  }
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------------------------------
__device__ void commit(const IllPassArgs& a, const PassHdr& H, PassLds& S) {
  CommitLds& C = S.cm;
  const uint32_t tag = tagof(H.epoch, a.W.layers);
  const int i = threadIdx.x;
  // every workgroup's partials (this also proves every workgroup has read the pass header)
  const bool ok = wg_wait([&]() {
    bool r = true;
    if (i < ILL_WG)
      for (int t = 0; t < 16; t++) r &= wok(aload64(a.lmp + (i * 16 + t) * 2), tag) & wok(aload64(a.lmp + (i * 16 + t) * 2 + 1), tag);
    return r;
  }, a.ctl, 700);
  if (!ok) return;
  trace_mark(a, 3 * ILL_MAXLAYERS + 4);
  for (int t = H.lmh0; t < H.lmh0 + H.lmhn; t++) {
    if (i < ILL_WG) {
      C.v[i] = wval(aload64(a.lmp + (i * 16 + t) * 2));
      C.i[i] = (int)(uint32_t)aload64(a.lmp + (i * 16 + t) * 2 + 1);
    }
    __syncthreads();
    for (int s = ILL_WG / 2; s >= 1; s >>= 1) {
      if (i < s) {
        float v = C.v[i];
        int id = C.i[i];
        amax_merge(v, id, C.v[i + s], C.i[i + s]);
        C.v[i] = v;
        C.i[i] = id;
      }
      __syncthreads();
    }
    if (i == 0) C.g[t] = C.i[0];
    __syncthreads();
  }
  IllState* st = a.st;
  if (i == 0) {
    C.npath = 0;
    C.pos0 = st->pos;
    if (H.commit == 0) {
      st->pos += H.nrows;
    } else if (H.commit == 1) {
      const int tok = C.g[H.lmh0];
      const int step = st->step;
      a.out_dev[step] = tok;
      __hip_atomic_store(a.out_host + step, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      st->step = step + 1;
      st->pos += H.nrows;
      st->n = 1;
      if (tok == st->eos0 || tok == st->eos1 || step + 1 >= st->maxsteps) st->done = 1;
      a.ptoks[0] = tok;
      a.ctl->last_tok = tok;
    } else {
      // speculative pass: rows 0..nrows-1 = [last token, drafts]; accept and commit
      const int nv = H.nrows;
      int m = 0;
      if (H.mode == ILL_MODE_TREE) {
        int cur = 0;
        for (;;) {
          int c = -1;
          for (int r = 1; r < nv; ++r)
            if (H.parent[r] == cur && H.tok[r] == C.g[cur]) { c = r; break; }
          if (c < 0) break;
          C.path[m++] = c;
          cur = c;
        }
      } else {
        while (m < nv - 1 && H.tok[m + 1] == C.g[m]) m++;
        for (int k = 0; k < m; k++) C.path[k] = k + 1;
      }
      st->passes += 1;
      st->accepted += m;
      bool stop = false;
      int last = C.g[0];
      for (int k = 0; k <= m && !stop; k++) {
        const int tok = C.g[k == 0 ? 0 : C.path[k - 1]];
        const int step = st->step;
        a.out_dev[step] = tok;
        __hip_atomic_store(a.out_host + step, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        st->step = step + 1;
        last = tok;
        if (tok == st->eos0 || tok == st->eos1 || step + 1 >= st->maxsteps) stop = true;
      }
      st->pos += m + 1;
      st->n = 1;
      st->nver = 1;
      st->tree = 0;
      if (stop) st->done = 1;
      a.ptoks[0] = last;
      a.ctl->last_tok = last;
      C.npath = H.mode == ILL_MODE_TREE ? m : 0;
    }
  }
  __syncthreads();
  // tree: accepted row path[k-1] (slot pos0 + path[k-1]) becomes slot pos0 + k; it was
  // already rotated as position pos0 + k (its depth). Sources never overlap destinations.
  const int np = C.npath;
  for (int k = 1; k <= np; k++) {
    const int src = C.pos0 + C.path[k - 1], dst = C.pos0 + k;
    if (src == dst) continue;
    const int NL = a.W.layers;
    for (int j = i; j < NL * ILL_NKV * 64; j += ILL_WG_THREADS) {
      const int lh = j >> 6, d = j & 63;
      uint16_t* kb = a.kc + (size_t)lh * a.maxctx * 64;
      kb[(size_t)dst * 64 + d] = kb[(size_t)src * 64 + d];
      uint16_t* vb = a.vt + (size_t)lh * (a.maxctx / 64) * 4096;
      vb[(size_t)(dst >> 6) * 4096 + d * 64 + (dst & 63)] = vb[(size_t)(src >> 6) * 4096 + d * 64 + (src & 63)];
    }
    __syncthreads();
  }
  if (i == 0) a.ctl->epoch = H.epoch + 1;
}

// ---------------------------------------------------------------------------------------
template <int T>
__global__ __launch_bounds__(ILL_WG_THREADS, 1) void ill_pass_kernel(IllPassArgs a) {
  __shared__ PassLds S;
  __shared__ PassHdr H;
  if (threadIdx.x == 0) {
    const IllState* st = a.st;
    const IllCtl* c = a.ctl;
    H.done = st->done;
    H.epoch = c->epoch;
    H.mode = c->mode;
    H.nrows = c->nrows;
    H.pos = st->pos;
    H.lmh0 = c->lmh_row0;
    H.lmhn = c->lmh_rows;
    H.wlog = c->write_logits;
    H.commit = c->commit;
    for (int t = 0; t < 16; t++) {
      H.tok[t] = t < H.nrows ? a.ptoks[t] : 0;
      if (H.mode == ILL_MODE_TREE) {
        H.depth[t] = t < H.nrows ? a.tree[ILL_TR_DEPTH + t] : 0;
        H.parent[t] = t < H.nrows ? a.tree[ILL_TR_PARENT + t] : 0;
      } else {
        H.depth[t] = t;
        H.parent[t] = t > 0 ? t - 1 : 0;
      }
    }
  }
  __syncthreads();
  if (H.done) return;
  const int wg = blockIdx.x;
  const int NL = a.W.layers;
  for (int l = 0; l < NL; l++) {
    bool ok = true;
    trace_mark(a, 3 * l);
    if (wg < ILL_R_QKV + ILL_NQB) ok = role_qkv<T>(a, H, S, l, wg - ILL_R_QKV);
    else if (wg >= ILL_R_ATT && wg < ILL_R_ATT + ILL_N_ATT) {
      const int nit = H.nrows * ILL_NKV;
      for (int it = wg - ILL_R_ATT; it < nit && ok; it += ILL_N_ATT) ok = role_att<T>(a, H, S, l, it & 1, it >> 1);
    } else if (wg >= ILL_R_O && wg < ILL_R_O + ILL_NOT) ok = role_o<T>(a, H, S, l, wg - ILL_R_O);
    else if (wg >= ILL_R_GUD && wg < ILL_R_GUD + ILL_NGU) ok = role_gud<T>(a, H, S, l, wg - ILL_R_GUD);
    else if (wg >= ILL_R_RED && wg < ILL_R_RED + ILL_NOT) ok = role_red<T>(a, H, l, wg - ILL_R_RED);
    if (!ok) return;
    trace_mark(a, 3 * l + 2);
  }
  trace_mark(a, 3 * ILL_MAXLAYERS);
  if (!role_lmh<T>(a, H, S)) return;
  trace_mark(a, 3 * ILL_MAXLAYERS + 2);
  if (wg == 0) {
    commit(a, H, S);
    trace_mark(a, 3 * ILL_MAXLAYERS + 5);
  }
}
