// Stand-alone q4 GEMV (the matrix-vector product of the decode step, measured on its own):
// y = W x for a q4 affine group-64 matrix W [rows][K] in the row-tile layout of the pass
// kernel, with the RMSNorm of x fused into the prologue (or a plain input, as the down
// projection takes) and an optional argmax epilogue (value, lowest index), as the lm_head
// uses it.
//
// Reference semantics: q4_chunk_norm / q_rows / reduce8 and k_lm_head_T
// (Sources/Engine/Shaders.swift:1001-1054, :1143-1185, :1327-1364). Arithmetic is the pass
// kernel's: x coded per 64-column group as 16-bit fixed point (int8 hi/lo), int8 MFMA
// against the nibbles (exact int32), fp32 group epilogue s*d*S + m*d*sum(v).
//
// Work split: a wave takes one (row tile, K slice) item and keeps the next item's weight
// loads in flight while it computes the current one. One slice per tile (the lm_head: many
// tiles): ill_gemv_q4_kernel, whose waves write y themselves. Several slices (the layer
// matrices: few tiles, so K is split to give every wave work): ill_gemv_q4_tiles_kernel,
// which places all slices of a tile in one workgroup and adds their fp32 partials in LDS in
// slice order (deterministic), with no second kernel. Both reduce the argmax per workgroup
// into key[par] (atomic max of order-preserving keys) and clear key[par ^ 1] for the next
// launch, which alternates par.
#pragma once
#include "ill_device.h"

#define ILL_GEMV_MAXG 128           // K <= 8192
#define ILL_GEMV_MAXBPS 8           // blocks (128 columns) per slice

struct IllGemvArgs {
  const uint8_t* w;      // [ntile][nb] 1 KiB blocks
  const uint32_t* s;     // [ntile][nb][16][2] (scale, min) f16 pairs
  const float* x;        // [K]
  const float* gamma;    // [K] or nullptr (plain input)
  int rows, K, bps, ks;  // blocks per slice, slices per tile (<= 8)
  float* y;              // [rows]
  uint64_t* key;         // argmax keys [2] (nullptr: no argmax); launch uses key[par]
  int par;
};

struct GemvLds {
  uint4 ahi[ILL_GEMV_MAXG * 4];
  uint4 alo[ILL_GEMV_MAXG * 4];
  float2 sc[ILL_GEMV_MAXG];
  float red[ILL_WAVES];
  uint64_t best[ILL_WAVES];
};

struct GemvItem {
  uint4 w[ILL_GEMV_MAXBPS];
  uint2 s[ILL_GEMV_MAXBPS];
};

template <bool ALL = false>
__device__ __forceinline__ void gemv_fetch(const IllGemvArgs& a, int item, int lane, GemvItem& it) {
  const int nb = a.K >> 7;
  const int tile = item / a.ks, slice = item - tile * a.ks;
  const int cb0 = slice * a.bps;
  const int n = lane & 15;
  // ALL: every block slot loads (slots past the slice reload its last block, unused): with
  // no branch between the loads, the compiler can wait for one item's loads while the next
  // item's stay in flight (the one-slice kernel, whose items fill the slots: lm_head 21.5
  // -> 19.6 us). Otherwise only the slice's blocks load (few-block items of split K).
#pragma unroll
  for (int i = 0; i < ILL_GEMV_MAXBPS; i++) {
    const int cb = min(cb0 + min(i, a.bps - 1), nb - 1);
    if (ALL || i < a.bps) {
      it.w[i] = gld((const uint4*)(a.w + ((size_t)tile * nb + cb) * 1024) + lane);
      it.s[i] = gld((const uint2*)(a.s + ((size_t)tile * nb + cb) * 32) + n);
    }
  }
}

// x: RMSNorm (sum of squares in a fixed order) and 16-bit coding per 64-column group into
// L (ends with a workgroup barrier).
__device__ __forceinline__ void gemv_prep_x(const IllGemvArgs& a, GemvLds& L) {
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int ng = a.K >> 6;
  float scale = 1.f;
  if (a.gamma) {
    float ss = 0.f;
    for (int c = tid; c < a.K; c += ILL_WG_THREADS) {
      const float v = gld(a.x + c);
      ss += v * v;
    }
    ss = gsum<64>(ss);
    if (lane == 0) L.red[w] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int ww = 0; ww < ILL_WAVES; ww++) tot += L.red[ww];
    scale = __builtin_amdgcn_rsqf(tot / (float)a.K + ILL_EPS);
  }
  for (int g = w; g < ng; g += ILL_WAVES) {
    const int c = 64 * g + lane;
    float v = gld(a.x + c);
    if (a.gamma) v = v * scale * gld(a.gamma + c);
    const float mx = gmax<64>(fabsf(v));
    const float d = mx * (1.0f / ILL_QMAX);
    const int qv = (int)rintf(v * (d > 0.f ? __builtin_amdgcn_rcpf(d) : 0.f));
    const int sq = gsumi<64>(qv);
    const int hi = (qv + 128) >> 8, lo = qv - (hi << 8);
    const int gi = lane >> 4;
    const int p = (lane & 8) | ((lane & 1) << 2) | ((lane >> 1) & 3);   // inverse of q4perm
    ((uint8_t*)&L.ahi[g * 4 + gi])[p] = (uint8_t)(hi & 0xff);
    ((uint8_t*)&L.alo[g * 4 + gi])[p] = (uint8_t)(lo & 0xff);
    if (lane == 0) L.sc[g] = make_float2(d, d * (float)sq);
  }
  __syncthreads();
}

// One item: the 16 row sums of its tile over its K slice (lane (kg, n) holds row n).
__device__ __forceinline__ float gemv_item(const IllGemvArgs& a, const GemvLds& L, const GemvItem& cur, int slice, int lane) {
  const int kg = lane >> 4;
  const int nb = a.K >> 7;
  const v4i z = {0, 0, 0, 0};
  const int cb0 = slice * a.bps;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < ILL_GEMV_MAXBPS; i++) {
    const int cb = cb0 + i;
    if (i < a.bps && cb < nb) {
#pragma unroll
      for (int gi = 0; gi < 2; gi++) {
        const int G = 2 * cb + gi;
        const v4i b = gi == 0 ? q4_unpack(cur.w[i].x, cur.w[i].y) : q4_unpack(cur.w[i].z, cur.w[i].w);
        const uint4 h = L.ahi[G * 4 + kg], l = L.alo[G * 4 + kg];
        const v4i ah = (v4i){(int)h.x, (int)h.y, (int)h.z, (int)h.w};
        const v4i al = (v4i){(int)l.x, (int)l.y, (int)l.z, (int)l.w};
        const v4i dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, b, z, 0, 0, 0);
        const v4i dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, b, z, 0, 0, 0);
        const uint32_t sm = gi == 0 ? cur.s[i].x : cur.s[i].y;
        const float2 dx = L.sc[G];
        const int S = (dh[0] << 8) + dl[0];
        acc = fmaf(h2f(sm & 0xffff), dx.x * (float)S, acc);
        acc = fmaf(h2f(sm >> 16), dx.y, acc);
      }
    }
  }
  return acc;
}

// One slice (ks == 1): every item is a whole tile; y and the argmax are written here.
__global__ __launch_bounds__(ILL_WG_THREADS, 1) void ill_gemv_q4_kernel(IllGemvArgs a) {
  __shared__ GemvLds L;
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int nitems = a.rows >> 4;   // one slice: an item is a whole tile
  const int stride = gridDim.x * ILL_WAVES;
  int item = blockIdx.x * ILL_WAVES + w;
  if (a.key && blockIdx.x == 0 && tid == 0) gst(a.key + (a.par ^ 1), (uint64_t)0);
  uint64_t kbest = 0;
  GemvItem cur;
  gemv_fetch<true>(a, min(item, nitems - 1), lane, cur);   // weights stream while x is prepared
  gemv_prep_x(a, L);
  while (item < nitems) {
    const int nxt = item + stride;
    GemvItem nx;
    gemv_fetch<true>(a, min(nxt, nitems - 1), lane, nx);   // unconditional (see gemv_fetch)
    const float acc = gemv_item(a, L, cur, 0, lane);
    if (kg == 0) {
      gst(a.y + 16 * item + n, acc);
      const uint64_t k = amax_key(acc, 16 * item + n);
      kbest = k > kbest ? k : kbest;
    }
    cur = nx;
    item = nxt;
  }
  if (a.key) {
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t ok = __shfl_xor(kbest, o, 64);
      kbest = ok > kbest ? ok : kbest;
    }
    if (lane == 0) L.best[w] = kbest;
    __syncthreads();
    if (tid == 0) {
      uint64_t m = L.best[0];
      for (int i = 1; i < ILL_WAVES; i++) m = L.best[i] > m ? L.best[i] : m;
      __hip_atomic_fetch_max((GAS unsigned long long*)(a.key + a.par), (unsigned long long)m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}


// Several slices per tile (ks <= 8): the ks slices of a tile are items of one workgroup, one
// per wave, so a round takes 8 / ks tiles; their fp32 partials meet in LDS and one wave per
// tile adds them in slice order, writes y and takes the argmax. Rounds step over the grid.
__global__ __launch_bounds__(ILL_WG_THREADS, 1) void ill_gemv_q4_tiles_kernel(IllGemvArgs a) {
  __shared__ GemvLds L;
  __shared__ float part[ILL_WAVES][16];   // [wave][row]
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int ntile = a.rows >> 4, ks = a.ks;
  const int tpr = ILL_WAVES / ks;
  const int nsets = (ntile + tpr - 1) / tpr;
  // this wave's item of round `set`, or -1
  auto item_of = [&](int set) -> int {
    const int tile = set * tpr + w / ks;
    return set < nsets && w < tpr * ks && tile < ntile ? tile * ks + w % ks : -1;
  };
  if (a.key && blockIdx.x == 0 && tid == 0) gst(a.key + (a.par ^ 1), (uint64_t)0);
  uint64_t kbest = 0;
  int set = blockIdx.x;
  int it = item_of(set);
  GemvItem cur;
  if (it >= 0) gemv_fetch(a, it, lane, cur);   // weights stream while x is prepared
  gemv_prep_x(a, L);
  for (; set < nsets; set += gridDim.x) {
    const int nx_it = item_of(set + gridDim.x);
    GemvItem nx;
    if (nx_it >= 0) gemv_fetch(a, nx_it, lane, nx);
    if (it >= 0) {
      const float acc = gemv_item(a, L, cur, w % ks, lane);
      if (kg == 0) part[w][n] = acc;
    }
    cur = nx;
    it = nx_it;
    __syncthreads();
    if (w < tpr && lane < 16) {
      const int tile = set * tpr + w;
      if (tile < ntile) {
        float v = 0.f;
        for (int sl = 0; sl < ks; sl++) v += part[w * ks + sl][lane];
        gst(a.y + 16 * tile + lane, v);
        const uint64_t k = amax_key(v, 16 * tile + lane);
        kbest = k > kbest ? k : kbest;
      }
    }
    __syncthreads();
  }
  if (a.key) {
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t ok = __shfl_xor(kbest, o, 64);
      kbest = ok > kbest ? ok : kbest;
    }
    if (lane == 0) L.best[w] = kbest;
    __syncthreads();
    if (tid == 0) {
      uint64_t m = L.best[0];
      for (int i = 1; i < ILL_WAVES; i++) m = L.best[i] > m ? L.best[i] : m;
      __hip_atomic_fetch_max((GAS unsigned long long*)(a.key + a.par), (unsigned long long)m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}
