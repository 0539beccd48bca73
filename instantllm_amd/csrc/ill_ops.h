// Layer-by-layer ("op") path: one kernel per operation, for any number of rows M.
//
// It serves what the persistent q4 pass kernel does not:
// * the prompt prefill in chunks of up to ILL_OP_MAXM rows, where the projections are real
//   GEMMs (M = 512 -> MFMA-bound), and
// * every pass of q8 and f16 models (decode steps, verify passes, prefill), whose per-layer
//   weights do not fit the persistent kernel's LDS stages.
//
// It follows the reference's own encoding (Engine.swift:370-403 encodePrefillLayer2 on
// gemm3_core, Shaders.swift:1911-2054; the 1-row kernels :1199-1364): per layer
//   norm(ln1) -> QKV GEMM (+bias, RoPE, K/V cache write) -> attention -> O GEMM (+x)
//   -> norm(ln2) -> gate/up GEMM (SiLU * up) -> down GEMM (+x),
// then the final norm and the lm_head GEMM with an argmax epilogue on the rows that need
// logits, and the commit.
//
// Arithmetic: activations in f16 (the reference's G3 path keeps fp16 activations too),
// weights dequantized to f16 in LDS (q4: s*q + m; q8: s*q; f16: as stored),
// v_mfma_f32_16x16x32_f16 with fp32 accumulation over K in a fixed order, fp32 residual
// stream. Every row's arithmetic is independent of M and of the rows beside it, so a row
// decoded alone and the same row inside a 16-row pass produce identical bits (the kernels
// are the same for M = 1 and M = 16; the 64-row tile is used only for prefill chunks).
//
// Every kernel reads the position and the stop flag from the device State, so a decode
// step recorded in a hipGraph replays correctly.
#pragma once
#include "ill_pass.h"

#define ILL_OP_MAXM 512

struct OpMat {
  const uint8_t* w;    // q4: codes [N][K/2]; q8: int8, f16: halves, both tiled (op_wt_off)
  const uint16_t* s;   // q4: [N][K/64][2] f16 (scale, min); q8: f16 tiled (op_st_off); f16: unused
  int N, K, qg;        // qg: q8 group size (32 or 64)
};

// The q8 and f16 matrices of the layer-by-layer path are tiled, so that a wave's 16-byte
// loads of one k-step (64 columns) read whole cache lines: 128-row blocks, k-steps, 16-row
// sub-tiles of 16 x 64 weights, inside which 16-byte units are ordered (8-column half e,
// 16-column group kg, row n). Element (r, k) of an N x K matrix of es-byte weights (N a
// multiple of 128, K of 64) lies at byte op_wt_off:
//   ((((r >> 7) * (K / 64) + (k >> 6)) * 8 + ((r & 127) >> 4)) * 64 es
//    + ((e * 4 + kg) * 16 + (r & 15)) * 16 + (k & 7) * es)   with kg = (k & 63) >> 4,
//   e = (k >> 3) & 1 for f16; for q8 a unit holds 16 columns (e = 0, (k & 15) bytes).
// A lane (kg, n) of op_fetch_b then reads 1 KB contiguous with its wave, and a thread of
// op_fetch_w (row, 32 columns) two 256-byte runs. q8 scales: [block][k-step][128 rows]
// [64 / qg] (op_st_off).
__host__ __device__ inline size_t op_wt_off(int r, int k, int K, int es) {
  const size_t tile = ((size_t)(r >> 7) * (K >> 6) + (k >> 6)) * 8 + ((r & 127) >> 4);
  const int kg = (k & 63) >> 4;
  if (es == 1) return tile * 1024 + (size_t)((kg * 16 + (r & 15)) * 16 + (k & 15));
  const int e = (k >> 3) & 1;
  return tile * 2048 + (size_t)(((e * 4 + kg) * 16 + (r & 15)) * 16 + (k & 7) * 2);
}
__host__ __device__ inline size_t op_st_off(int r, int k, int K, int qg) {
  return (((size_t)(r >> 7) * (K >> 6) + (k >> 6)) * 128 + (r & 127)) * (64 / qg) + ((k & 63) / qg);
}

struct OpLayerW {
  OpMat qkv, o, gu, d;
  // W_o again, head-major for the O projection folded into attention (q8 / f16): codes
  // [head][16-byte column chunk][896 rows] (4 chunks q8, 8 f16), scales (q8) [head][896 rows]
  // as u32 (scale of k 0-31 | scale of k 32-63 << 16), so that a lane per row reads
  // consecutive 16 bytes
  OpMat oh;
  const float* bqkv;
  const float* ln1;
  const float* ln2;
};

struct OpCtx {
  const OpLayerW* L;
  OpMat emb;             // embedding = tied lm_head
  const float* fnorm;
  IllState* st;
  IllCtl* ctl;
  int32_t* ptoks;        // [M] row tokens (commit writes [0])
  const int32_t* tree;   // [65]
  const float2* rope;
  uint16_t* kc;
  uint16_t* vt;
  float* x;              // [M][896] residual stream
  __half* xn;            // [M][896] normalized activations
  float* q;              // [M][896] queries
  __half* ao;            // [M][896] attention output
  __half* h;             // [M][4864] SiLU(gate) * up
  uint64_t* amax;        // [V/128][16] argmax keys of the lm_head tiles
  float* logits;         // [16][V]
  int maxctx, layers, vocab;
  int kvswz;             // K/V cache layout: 1 swizzled (q8 / f16), 0 rows (q4; ill_common.h)
};

// What the kernels need from the State and the control block, read once at kernel entry
// together with their first operands (a load that gates the others would add a memory round
// trip to every kernel); `done` is checked before the first store.
struct OpHdr {
  int done, pos, mode, wlog;
};
__device__ __forceinline__ OpHdr op_hdr(const OpCtx& c) {
  OpHdr h;
  h.done = gld(&c.st->done);
  h.pos = gld(&c.st->pos);
  h.mode = gld(&c.ctl->mode);
  h.wlog = gld(&c.ctl->write_logits);
  return h;
}

// Row t's position offset from pos (its depth): tree passes read the tree, others are chains.
__device__ __forceinline__ int op_depth(const OpCtx& c, int mode, int t) {
  return mode == ILL_MODE_TREE ? gld(c.tree + ILL_TR_DEPTH + t) : (mode == ILL_MODE_DECODE ? 0 : t);
}

// ---- embedding and RMSNorm -----------------------------------------------------------
template <int FMT>
__device__ __forceinline__ float op_dequant1(const OpMat& m, int r, int k) {
  if constexpr (FMT == 2) {
    const uint8_t b = m.w[(size_t)r * (m.K / 2) + k / 2];
    const float q = (float)((k & 1) ? (b >> 4) : (b & 15));
    const uint32_t sm = *(const uint32_t*)(m.s + ((size_t)r * (m.K / 64) + k / 64) * 2);
    return h2f(sm & 0xffff) * q + h2f(sm >> 16);
  } else if constexpr (FMT == 1) {
    const float q = (float)(int8_t)m.w[op_wt_off(r, k, m.K, 1)];
    return h2f(m.s[op_st_off(r, k, m.K, m.qg)]) * q;
  } else {
    return h2f(*(const uint16_t*)(m.w + op_wt_off(r, k, m.K, 2)));
  }
}

// x[t][:] = embedding row of ptoks[t] (Shaders.swift:118-126, :179-190)

// xn[t] = f16(x[t] * rsqrt(mean(x^2) + eps) * gamma) for rows row0 .. row0 + M - 1 (one wave
// per row; sum of squares in a fixed order). Output row index t - row0.
__global__ __launch_bounds__(256) void op_norm_kernel(OpCtx c, const float* gamma, int row0, int M) {
  const int done = gld(&c.st->done);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + w;
  if (t >= M) return;
  const float* xr = c.x + (size_t)(row0 + t) * ILL_H;
  float v[14], g[14];
#pragma unroll
  for (int i = 0; i < 14; i++) {
    v[i] = gld(xr + 64 * i + lane);
    g[i] = gld(gamma + 64 * i + lane);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 14; i++) ss += v[i] * v[i];
  ss = gsum<64>(ss);
  const float scale = __builtin_amdgcn_rsqf(ss * (1.0f / (float)ILL_H) + ILL_EPS);
  if (done) return;
#pragma unroll
  for (int i = 0; i < 14; i++)
    gst((uint16_t*)(c.xn + (size_t)t * ILL_H + 64 * i + lane), (uint16_t)__half_as_ushort(__float2half(v[i] * scale * g[i])));
}

// The embedding rows of the pass's tokens into x and, from the same registers, layer 0's
// RMSNorm of them into xn, in one launch (one wave per row; the sum of squares in
// op_norm_kernel's order).
template <int FMT>
__global__ __launch_bounds__(256) void op_embed_norm_kernel(OpCtx c, const float* gamma, int M) {
  const int done = gld(&c.st->done);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + w;
  if (t >= M) return;
  const int tok = gld(c.ptoks + t);
  float v[14], g[14];
#pragma unroll
  for (int i = 0; i < 14; i++) {
    v[i] = op_dequant1<FMT>(c.emb, tok, 64 * i + lane);
    g[i] = gld(gamma + 64 * i + lane);
  }
  float* xr = c.x + (size_t)t * ILL_H;
  if (!done) {
#pragma unroll
    for (int i = 0; i < 14; i++) gst(xr + 64 * i + lane, v[i]);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 14; i++) ss += v[i] * v[i];
  ss = gsum<64>(ss);
  const float scale = __builtin_amdgcn_rsqf(ss * (1.0f / (float)ILL_H) + ILL_EPS);
  if (done) return;
#pragma unroll
  for (int i = 0; i < 14; i++)
    gst((uint16_t*)(c.xn + (size_t)t * ILL_H + 64 * i + lane), (uint16_t)__half_as_ushort(__float2half(v[i] * scale * g[i])));
}

// ---- GEMM: Y[M][N] = A[M][K] (f16) * W[N][K]^T, fused epilogues ------------------------
enum OpEpi { OP_QKV = 0, OP_RESID = 1, OP_SILU = 2, OP_LMH = 3 };

struct OpGemmArgs {
  OpCtx c;
  const __half* A;   // [M][K]
  OpMat W;
  int M, layer;
  float* resid;      // OP_RESID: [M][896] += Y
  float* part;       // split K: [slices][M][N] fp32 partials
  int ksteps;        // 64-column steps per K slice
  const float* apart;   // op_gemv_kernel<.., SILU = true>: gate/up partials [aS][M][2K]
  int aS;
  int pos_hint;         // the State's pos as the host expects it (QKV epilogue: rotary rows
                        // are loaded for pos_hint + row with the partials)
};

#define OP_BN 128
#define OP_BK 64
#define OP_LDK 72    // LDS row stride in halves (padding against bank conflicts)
#define OP_MAXS 24   // K slices of a split GEMM at most

// One k-step (64 columns) of the weight tile, rows n0 .. n0+127, as loaded from HBM, and
// its dequantization into LDS [128][OP_LDK] f16. Thread -> (row tid / 2, half tid % 2).
template <int FMT>
struct WRaw {
  uint4 b[FMT == 2 ? 1 : (FMT == 1 ? 2 : 4)];
  // q4: (scale, min) pair; q8: the scale, kept 16-bit so that the load needs no widening
  // (which would wait for it at once)
  std::conditional_t<FMT == 1, uint16_t, uint32_t> sm;
};

template <int FMT>
__device__ __forceinline__ void op_fetch_w(const OpMat& W, int n0, int k0, int tid, WRaw<FMT>& r) {
  const int row = n0 + (tid >> 1), hf = tid & 1;
  if constexpr (FMT == 2) {
    r.b[0] = gld((const uint4*)(W.w + (size_t)row * (W.K / 2) + k0 / 2 + 16 * hf));
    r.sm = gld((const uint32_t*)(W.s + ((size_t)row * (W.K / 64) + k0 / 64) * 2));
  } else if constexpr (FMT == 1) {
    r.b[0] = gld((const uint4*)(W.w + op_wt_off(row, k0 + 32 * hf, W.K, 1)));
    r.b[1] = gld((const uint4*)(W.w + op_wt_off(row, k0 + 32 * hf + 16, W.K, 1)));
    r.sm = gld(W.s + op_st_off(row, k0 + 32 * hf, W.K, W.qg));
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) r.b[i] = gld((const uint4*)(W.w + op_wt_off(row, k0 + 32 * hf + 8 * i, W.K, 2)));
  }
}

// q8 dequantization, 4 weights at a time: s * (f16)q for the 4 int8 codes of x. Each code
// q becomes the half 1024 + (q + 128) (exponent 0x64 over the byte q ^ 0x80, built with
// v_perm), from which 1152 is subtracted: both exact, so the products equal
// s * (_Float16)(float)q, computed two at a time on packed f16 (v_pk_add_f16, v_pk_mul_f16).
typedef _Float16 op_h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void op_q8x4(uint32_t x, _Float16 s, _Float16* o) {
  const uint32_t u = x ^ 0x80808080u;
  const op_h2 k = {(_Float16)1152.f, (_Float16)1152.f}, sc = {s, s};
  const op_h2 a = __builtin_bit_cast(op_h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - k;
  const op_h2 b = __builtin_bit_cast(op_h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - k;
  const op_h2 pa = a * sc, pb = b * sc;
  o[0] = pa[0];
  o[1] = pa[1];
  o[2] = pb[0];
  o[3] = pb[1];
}

template <int FMT>
__device__ __forceinline__ void op_store_w(const WRaw<FMT>& r, _Float16* Bs, int tid) {
  _Float16* dst = Bs + (tid >> 1) * OP_LDK + 32 * (tid & 1);
  if constexpr (FMT == 2) {
    const _Float16 s = (_Float16)h2f(r.sm & 0xffff), m = (_Float16)h2f(r.sm >> 16);
    const uint32_t x[4] = {r.b[0].x, r.b[0].y, r.b[0].z, r.b[0].w};
    _Float16 o[32];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t byte = (x[i >> 2] >> (8 * (i & 3))) & 0xff;
      o[2 * i] = s * (_Float16)(float)(byte & 15) + m;
      o[2 * i + 1] = s * (_Float16)(float)(byte >> 4) + m;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) *(uint4*)(dst + 8 * i) = *(const uint4*)(o + 8 * i);
  } else if constexpr (FMT == 1) {
    const _Float16 s = (_Float16)h2f(r.sm);
    const uint32_t x[8] = {r.b[0].x, r.b[0].y, r.b[0].z, r.b[0].w, r.b[1].x, r.b[1].y, r.b[1].z, r.b[1].w};
    _Float16 o[32];
#pragma unroll
    for (int i = 0; i < 8; i++) op_q8x4(x[i], s, o + 4 * i);
#pragma unroll
    for (int i = 0; i < 4; i++) *(uint4*)(dst + 8 * i) = *(const uint4*)(o + 8 * i);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) *(uint4*)(dst + 8 * i) = r.b[i];
  }
}

// A tile: BM rows x 64 halves; thread i (< BM * 8) carries 16 bytes (rows >= M read row
// M - 1: finite, and their outputs are unused). Every thread loads (the surplus ones a
// duplicate), so that the number of loads in flight never depends on a branch.
template <int BM>
struct ARaw {
  uint4 v[(BM * 8 + 255) / 256];
};
template <int BM>
__device__ __forceinline__ void op_fetch_a(const __half* A, int M, int K, int m0, int k0, int tid, ARaw<BM>& r) {
#pragma unroll
  for (int u = 0; u < (BM * 8 + 255) / 256; u++) {
    const int i = (tid + 256 * u) & (BM * 8 - 1);
    const int row = min(m0 + (i >> 3), M - 1);
    r.v[u] = gld((const uint4*)(A + (size_t)row * K + k0) + (i & 7));
  }
}
template <int BM>
__device__ __forceinline__ void op_store_a(const ARaw<BM>& r, _Float16* As, int tid) {
#pragma unroll
  for (int u = 0; u < (BM * 8 + 255) / 256; u++) {
    const int i = tid + 256 * u;
    if (i < BM * 8) *(uint4*)(As + (i >> 3) * OP_LDK + 8 * (i & 7)) = r.v[u];
  }
}

// ---- epilogues (shared by the fused GEMM and the split-K reduction) ---------------------
// QKV: one rotary block b = columns 32 b .. +31 holds dims d (x0, columns 32 b + i) and
// d + 32 (x1, columns 32 b + 16 + i) of head b / 2 (Convert.swift:236-244); q heads 0-13,
// k 14-15, v 16-17: bias, RoPE at the row's position, then q or the K / V cache slot.
// cs_at / cs: a rotary row already loaded for position cs_at (-1: none), used when it is
// the row's position; bpre: the two bias values already loaded (nullptr: load them).
__device__ __forceinline__ void epi_qkv(const OpCtx& c, const OpHdr& hd, int layer, int m, int b, int i, float x0, float x1,
                                        int cs_at = -1, float2 cs_pre = make_float2(0.f, 0.f), const float* bpre = nullptr) {
  const int head = b >> 1, d = (b & 1) * 16 + i;
  x0 += bpre ? bpre[0] : gld(c.L[layer].bqkv + 32 * b + i);
  x1 += bpre ? bpre[1] : gld(c.L[layer].bqkv + 32 * b + 16 + i);
  const int pos = hd.pos;
  if (head < ILL_NH + ILL_NKV) {
    const int p = pos + op_depth(c, hd.mode, m);
    const float2 cs = p == cs_at ? cs_pre : gld(c.rope + p * 32 + d);
    const float r0 = x0 * cs.x - x1 * cs.y, r1 = x1 * cs.x + x0 * cs.y;
    x0 = r0;
    x1 = r1;
  }
  const int slot = pos + m;
  if (head < ILL_NH) {
    c.q[(size_t)m * ILL_H + head * 64 + d] = x0;
    c.q[(size_t)m * ILL_H + head * 64 + d + 32] = x1;
  } else if (head < ILL_NH + ILL_NKV) {
    uint16_t* kb = c.kc + ((size_t)layer * ILL_NKV + (head - ILL_NH)) * c.maxctx * 64;
    kb[kv_k_off(slot, d, c.kvswz)] = (uint16_t)f2h(x0);
    kb[kv_k_off(slot, d + 32, c.kvswz)] = (uint16_t)f2h(x1);
  } else {
    uint16_t* vb = c.vt + ((size_t)layer * ILL_NKV + (head - ILL_NH - ILL_NKV)) * (c.maxctx / 64) * 4096;
    vb[kv_v_off(slot, d, c.kvswz)] = (uint16_t)f2h_sat(x0);
    vb[kv_v_off(slot, d + 32, c.kvswz)] = (uint16_t)f2h_sat(x1);
  }
}
// gate/up rows in groups of 4: g[2q], g[2q+1], u[2q], u[2q+1] (Convert.swift:134-136)
__device__ __forceinline__ void epi_silu(const OpCtx& c, int m, int unit, float g, float u) {
  c.h[(size_t)m * ILL_FF + unit] = __float2half(g / (1.0f + expf(-g)) * u);
}

// Epilogue of a 128-column tile (lane (kg, n) of wave w holds rows m0 + 16 i + 4 kg + r,
// columns n0 + 32 w + 16 j + n): fp32 partials of a K slice, or the fused epilogue.
// QKV: cs_base >= 0 gives the rotary rows cs[4 i + r] of rows m0 + 16 i + 4 kg + r at
// position cs_base + row (used when that is the row's position); qbias: the lane's two bias
// values, already loaded (nullptr: loaded here).
template <int BM, int EPI>
__device__ __forceinline__ void op_gemm_epilogue(const OpGemmArgs& a, const OpHdr& hd, const v4f (&acc)[BM / 16][2], int m0,
                                                 int n0, int kz, int w, int kg, int n, uint64_t (&red)[4][16],
                                                 int cs_base = -1, const float2* cs = nullptr, const float* qbias = nullptr) {
  constexpr int TM = BM / 16;
  if (hd.done) return;
  const OpCtx& c = a.c;
  const int tid = threadIdx.x;
  if (gridDim.z > 1) {   // split K: partials for op_epi_kernel
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = m0 + 16 * i + 4 * kg + r, col = n0 + 32 * w + 16 * j + n;
          if (m < a.M) a.part[((size_t)kz * a.M + m) * a.W.N + col] = acc[i][j][r];
        }
    return;
  }
  // ---- fused epilogues: lane holds rows 16 i + 4 kg + r, columns n0 + 32 w + 16 j + n
  if constexpr (EPI == OP_RESID) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = m0 + 16 * i + 4 * kg + r, col = n0 + 32 * w + 16 * j + n;
          if (m < a.M) a.resid[(size_t)m * ILL_H + col] += acc[i][j][r];
        }
  } else if constexpr (EPI == OP_SILU) {
    // Lanes n % 4 = 0, 1 hold the gate values of units 2 q, 2 q + 1 and lanes 2, 3 their up
    // values. The quad's halves swap rows (quad_perm 2 3 0 1): lanes 0, 1 then apply rows
    // 4 kg + 0, 1 and lanes 2, 3 rows 4 kg + 2, 3, so that every lane computes two units.
    const bool lo = (n & 3) < 2;
    const int u = (n & 3) - (lo ? 0 : 2);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int col = n0 + 32 * w + 16 * j + n;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const float mine = acc[i][j][lo ? h : 2 + h], send = acc[i][j][lo ? 2 + h : h];
          const float got = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), 0x4e, 0xf, 0xf, false));
          const int m = m0 + 16 * i + 4 * kg + (lo ? h : 2 + h);
          if (m < a.M) epi_silu(c, m, (col >> 2) * 2 + u, lo ? mine : got, lo ? got : mine);
        }
      }
  } else if constexpr (EPI == OP_QKV) {
    const int b = (n0 + 32 * w) >> 5;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + 16 * i + 4 * kg + r;
        if (m < a.M) {
          if (cs_base >= 0) epi_qkv(c, hd, a.layer, m, b, n, acc[i][0][r], acc[i][1][r], cs_base + m, cs[4 * i + r], qbias);
          else epi_qkv(c, hd, a.layer, m, b, n, acc[i][0][r], acc[i][1][r], -1, make_float2(0.f, 0.f), qbias);
        }
      }
  } else {   // OP_LMH: logits (optional) and per-tile argmax keys per row (BM == 16)
    const int wlog = hd.wlog;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = 4 * kg + r;
      uint64_t k = 0;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int col = n0 + 32 * w + 16 * j + n;
        const float v = acc[0][j][r];
        if (wlog && m < a.M) c.logits[(size_t)m * c.vocab + col] = v;
        const uint64_t kk = amax_key(v, col);
        k = kk > k ? kk : k;
      }
      for (int o = 8; o >= 1; o >>= 1) {
        const uint64_t ok = __shfl_xor(k, o, 64);
        k = ok > k ? ok : k;
      }
      if (n == 0) red[w][m] = k;
    }
    __syncthreads();
    if (tid < 16) {
      uint64_t k = red[0][tid];
      for (int ww = 1; ww < 4; ww++) k = red[ww][tid] > k ? red[ww][tid] : k;
      c.amax[(size_t)blockIdx.x * 16 + tid] = k;
    }
  }
}

// Workgroup: 256 threads = 4 waves; a wave owns 32 columns (two 16-column MFMA tiles) of
// the 128-column tile and all BM rows. blockIdx.z selects a K slice of `ksteps` 64-column
// steps; with more than one slice the kernel writes fp32 partials [slice][M][N] and
// op_epi_kernel reduces them in slice order and applies the epilogue.
// DEPTH > 1: the operands of the next DEPTH k-steps are in flight (a register ring) while
// the current one is multiplied, and the LDS tiles are double-buffered, so one barrier per
// k-step orders both their reuse and their filling; it waits for LDS traffic only (a full
// __syncthreads would also drain the ring's loads). DEPTH 1: one k-step ahead, one LDS
// buffer, two barriers per k-step, half the LDS and fewer registers: more workgroups per
// CU, which is what the many-tile prefill gate/up GEMM needs (25.6 vs 40.7 us at 512 rows,
// f16), while the ring wins where the tiles are few (O and down: 14.6 vs 17.0 us).
// Tile of a prefill GEMM workgroup (grid: column tiles x row tiles x K slices). Workgroups
// are dealt to the 8 XCDs round-robin (workgroup id mod 8), and each XCD has its own L2, so
// the tiles are renumbered: the order (K slice, column tile, row tile) is cut into 8
// contiguous runs, run c going to the workgroups on XCD c in dispatch order. The row tiles
// of a weight slab (column tile, K slice) then share one XCD's L2 instead of fetching the
// slab from HBM once per XCD (512-row down projection, f16: 19.3 -> 16.5 us; QKV and O
// 2-7% faster). A permutation of tiles: the results do not change.
struct OpTile {
  int x, y, z;
};
__device__ __forceinline__ OpTile op_tile_xcd() {
  const int nx = gridDim.x, ny = gridDim.y;
  const int T = nx * ny * gridDim.z;
  const int id = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
  const int c = id & 7, k = id >> 3;
  const int u = c * (T >> 3) + min(c, T & 7) + k;   // XCD c holds ceil((T - c) / 8) workgroups
  const int y = u % ny, sl = u / ny;
  return {sl % nx, y, sl / nx};
}

template <int FMT, int BM, int EPI, int DEPTH, int NB = (DEPTH > 1 ? 2 : 1)>
__global__ __launch_bounds__(256) void op_gemm_kernel(OpGemmArgs a) {
  const OpHdr hd = op_hdr(a.c);
  __shared__ __attribute__((aligned(16))) _Float16 As[NB][BM * OP_LDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[NB][OP_BN * OP_LDK];
  __shared__ uint64_t red[4][16];
  constexpr int TM = BM / 16;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  // (the gate/up GEMM keeps the dispatch order: renumbered it ran 1.5-10% slower, measured)
  const OpTile tl = BM == 64 && EPI != OP_SILU ? op_tile_xcd() : OpTile{(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z};
  const int n0 = tl.x * OP_BN, m0 = tl.y * BM;
  const int K = a.W.K;
  const int kb = tl.z * a.ksteps * OP_BK, ke = min(K, kb + a.ksteps * OP_BK);
  const int ns = (ke - kb) / OP_BK;
  v4f acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; i++) {
    acc[i][0] = (v4f){0.f, 0.f, 0.f, 0.f};
    acc[i][1] = (v4f){0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (DEPTH == 1) {
    WRaw<FMT> wr;
    ARaw<BM> ar;
    op_fetch_w<FMT>(a.W, n0, kb, tid, wr);
    op_fetch_a<BM>(a.A, a.M, K, m0, kb, tid, ar);
    for (int k0 = kb; k0 < ke; k0 += OP_BK) {
      op_store_a<BM>(ar, As[0], tid);
      op_store_w<FMT>(wr, Bs[0], tid);
      __syncthreads();
      if (k0 + OP_BK < ke) {
        op_fetch_w<FMT>(a.W, n0, k0 + OP_BK, tid, wr);
        op_fetch_a<BM>(a.A, a.M, K, m0, k0 + OP_BK, tid, ar);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        v8h bf[2];
#pragma unroll
        for (int j = 0; j < 2; j++) bf[j] = *(const v8h*)(Bs[0] + (32 * w + 16 * j + n) * OP_LDK + 32 * ks + 8 * kg);
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const v8h af = *(const v8h*)(As[0] + (16 * i + n) * OP_LDK + 32 * ks + 8 * kg);
#pragma unroll
          for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
        }
      }
      __syncthreads();
    }
    op_gemm_epilogue<BM, EPI>(a, hd, acc, m0, n0, tl.z, w, kg, n, red);
    return;
  }
  constexpr int OP_DEPTH = DEPTH;
  // Ring loads are unconditional (steps past the slice reload its last one), so that the
  // compiler can count the loads in flight and wait for the oldest slot only.
  WRaw<FMT> wr[OP_DEPTH];
  ARaw<BM> ar[OP_DEPTH];
#pragma unroll
  for (int d = 0; d < OP_DEPTH; d++) {
    const int k0 = kb + min(d, ns - 1) * OP_BK;
    op_fetch_w<FMT>(a.W, n0, k0, tid, wr[d]);
    op_fetch_a<BM>(a.A, a.M, K, m0, k0, tid, ar[d]);
    __builtin_amdgcn_sched_barrier(0);   // issue order = slot order (the waits count on it)
  }
  // One k-step from ring slot d (st: the step's index in the slice); `refetch` refills the
  // slot with step st + OP_DEPTH (clamped: the last round reloads the slice's last step).
  auto kstep = [&](int d, int st, bool refetch) {
    _Float16* as = As[(d & 1) % NB];
    _Float16* bs = Bs[(d & 1) % NB];
    if constexpr (NB == 1) lds_barrier();   // one buffer: every wave is done with the last step
    op_store_a<BM>(ar[d], as, tid);
    op_store_w<FMT>(wr[d], bs, tid);
    lds_barrier();   // LDS only: the ring's HBM loads stay in flight
    if (refetch) {
      const int k0 = kb + min(st + OP_DEPTH, ns - 1) * OP_BK;
      __builtin_amdgcn_sched_barrier(0);
      op_fetch_w<FMT>(a.W, n0, k0, tid, wr[d]);
      op_fetch_a<BM>(a.A, a.M, K, m0, k0, tid, ar[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      v8h bf[2];
#pragma unroll
      for (int j = 0; j < 2; j++) bf[j] = *(const v8h*)(bs + (32 * w + 16 * j + n) * OP_LDK + 32 * ks + 8 * kg);
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const v8h af = *(const v8h*)(as + (16 * i + n) * OP_LDK + 32 * ks + 8 * kg);
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
  };
  // Whole rounds of OP_DEPTH steps with no branch between their loads (so every path into
  // the loop head has the same loads in flight and the waits stay partial), then the tail
  // from the ring without refills.
  int s0 = 0;
  for (; s0 + OP_DEPTH <= ns; s0 += OP_DEPTH) {
#pragma unroll
    for (int d = 0; d < OP_DEPTH; d++) kstep(d, s0 + d, true);
  }
#pragma unroll
  for (int d = 0; d < OP_DEPTH - 1; d++)
    if (s0 + d < ns) kstep(d, s0 + d, false);
  op_gemm_epilogue<BM, EPI>(a, hd, acc, m0, n0, tl.z, w, kg, n, red);
}

// ---- prefill GEMM, q8 / f16: operands streamed from memory into an LDS ring --------------
// op_gemm_kernel stages the next k-step (64 columns) in registers, one step ahead (DEPTH 1)
// or a ring of DEPTH steps, and stores it to LDS. Here the operands go from memory straight
// into LDS (global_load_lds_dwordx4: lane i of a wave's load writes 16 bytes at the
// instruction's LDS address + 16 i), into a ring of ST stages, so that ST - 1 k-steps are in
// flight with no registers or LDS stores spent on them. (Per workgroup at 512 rows: 0.7 us
// to issue the prologue, then 0.3-0.7 us per k-step; the gate/up GEMM, three workgroups per
// CU, is bound by the LDS traffic of its k-steps: 24 KB written and 48 KB read, the four
// waves reading the same A rows.) A stage holds
//   A: BM rows x 64 halves in 16-byte units ordered (row / 16, k / 8, row % 16), so that the
//      16 lanes of an MFMA operand read 256 contiguous bytes (no bank conflicts);
//   B: the k-step's block of the tiled weights (128 rows x 64 columns at op_wt_off, 8 KB q8,
//      16 KB f16) as stored: its units are already in that order;
//   q8: the block's scales (128 rows x 64 / qg f16, op_st_off), 256 or 512 bytes.
// q8 weights are dequantized as they leave LDS, with op_store_w's arithmetic, and every
// output sums the same products in the same order as op_gemm_kernel: the results are
// identical. The loads are issued in inline assembly: the compiler's own tracking of LDS
// loads in flight made it wait for all of them before some of the stage's LDS reads (it
// could not tell the stages apart), which serialized the ring. The wait for the stage about
// to be read is explicit: vmcnt counts this wave's own loads, and the barrier after it covers
// the other waves' loads and orders every wave's reads of the stage refilled next before the
// refill. (The compiler's waits for its own loads count only the loads it knows of, so they
// wait at least as long as they need: loads complete in issue order.)
#define OP_LDS(p) ((__attribute__((address_space(3))) void*)(p))
// One wave-wide load into LDS: lane i's `bytes` (16 or 4) at global g go to LDS byte address
// lds + bytes * i (lds: the same for every lane).
__device__ __forceinline__ void op_lds_dma16(const void* g, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)OP_LDS(lds));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m), "v"(g) : "m0");
}
__device__ __forceinline__ void op_lds_dma4(const void* g, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)OP_LDS(lds));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(m), "v"(g) : "m0");
}
// Stages: 24 KB (f16) / 16.5 KB (q8) each at BM 64, 20 / 12.5 KB at BM 32. Rings of 6 (f16)
// and 8 (q8) stages for the GEMMs of at most one workgroup per CU, and for all of them, were
// slower (512-row prefill 1.96 / 2.24 ms against 1.93 / 2.12 ms; 2.17 / 2.55 ms): issuing the
// longer prologue took 2 us instead of 0.7 and the k-steps were hardly faster. The gate/up
// GEMM (608 workgroups at 512 rows) takes 2 (f16) / 3 (q8) stages, so that three workgroups
// fit per CU and all of them run in one round (f16: 1.90 -> 1.86 ms).
#define OP_RING_ST(FMT, EPI) ((EPI) == OP_SILU ? ((FMT) == 0 ? 2 : 3) : ((FMT) == 0 ? 3 : 4))
template <int FMT, int BM>
struct OpRing {                                  // sizes in 16-byte units
  static constexpr int A = BM * 8;
  static constexpr int B = FMT == 0 ? 1024 : 512;
  static constexpr int SC = FMT == 1 ? 32 : 0;
  static constexpr int N = A + B + SC;
  static constexpr int LA = A >= 256 ? A / 256 : 1;   // A loads per thread (BM 16: waves 2, 3 repeat 0, 1)
  static constexpr int L = LA + B / 256 + (FMT == 1 ? 1 : 0);   // loads per thread and stage
};

// Thread tid's loads of the k-step at k0 into stage st (rows >= M read row M - 1).
template <int FMT, int BM>
__device__ __forceinline__ void op_ring_load(const OpGemmArgs& a, int m0, int n0, int k0, uint4* st, int tid) {
  using R = OpRing<FMT, BM>;
  const int K = a.W.K, wb = tid & ~63;   // wave's first unit of each 256-unit run
#pragma unroll
  for (int u = 0; u < R::LA; u++) {
    // unit p (BM 16: 128 units, which waves 2, 3 load again into the same bytes, so that every
    // wave issues the same loads)
    const int p = (256 * u + tid) & (R::A - 1);
    const int row = min(m0 + ((p >> 7) << 4) + (p & 15), a.M - 1);
    op_lds_dma16(a.A + (size_t)row * K + k0 + 8 * ((p >> 4) & 7), st + ((256 * u + wb) & (R::A - 1)));
  }
  const uint4* blk = (const uint4*)(a.W.w + op_wt_off(n0, k0, K, FMT == 0 ? 2 : 1));
#pragma unroll
  for (int u = 0; u < R::B / 256; u++)
    op_lds_dma16(blk + 256 * u + tid, st + R::A + 256 * u + wb);
  if constexpr (FMT == 1) {   // 64 dwords per wave: all of them (qg 64), or half (qg 32: waves 0, 2 the first)
    const int off = a.W.qg == 32 ? ((tid >> 6) & 1) * 64 : 0;
    const uint32_t* sc = (const uint32_t*)(a.W.s + op_st_off(n0, k0, K, a.W.qg));
    op_lds_dma4(sc + off + (tid & 63), (uint32_t*)(st + R::A + R::B) + off);
  }
}

// The k-step in stage st: lane (kg, n) of wave w, rows 16 i + n, columns 32 w + 16 j + n.
template <int FMT, int BM>
__device__ __forceinline__ void op_ring_mma(const uint4* st, int w, int kg, int n, int qg, v4f (&acc)[BM / 16][2]) {
  using R = OpRing<FMT, BM>;
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    v8h bf[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int c16 = 2 * w + j;   // 16-row sub-tile of the weight block
      if constexpr (FMT == 0) {
        bf[j] = u4_to_v8h(st[R::A + c16 * 128 + ((kg & 1) * 4 + 2 * ks + (kg >> 1)) * 16 + n]);
      } else {
        const uint2 q = ((const uint2*)(st + R::A + c16 * 64 + (2 * ks + (kg >> 1)) * 16 + n))[kg & 1];
        const uint16_t* sc = (const uint16_t*)(st + R::A + R::B);
        const _Float16 s = (_Float16)h2f(sc[(16 * c16 + n) * (64 / qg) + (qg == 32 ? ks : 0)]);
        _Float16 o[8];
        op_q8x4(q.x, s, o);
        op_q8x4(q.y, s, o + 4);
#pragma unroll
        for (int i = 0; i < 8; i++) bf[j][i] = o[i];
      }
    }
#pragma unroll
    for (int i = 0; i < BM / 16; i++) {
      const v8h af = u4_to_v8h(st[i * 128 + (4 * ks + kg) * 16 + n]);
#pragma unroll
      for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
    }
  }
}

// Wait until at most `later` stages of this wave's loads are in flight (a constant once the
// callers' loops are unrolled), then the workgroup barrier.
template <int N>
__device__ __forceinline__ void op_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
template <int L>
__device__ __forceinline__ void op_ring_wait(int later) {
  switch (later) {
    case 0: op_vm_barrier<0>(); break;
    case 1: op_vm_barrier<L>(); break;
    case 2: op_vm_barrier<2 * L>(); break;
    case 3: op_vm_barrier<3 * L>(); break;
    case 4: op_vm_barrier<4 * L>(); break;
    case 5: op_vm_barrier<5 * L>(); break;
    default: op_vm_barrier<6 * L>(); break;
  }
}

// Grid, tiles and epilogues as op_gemm_kernel (4 waves; wave w owns columns 32 w .. + 31 of
// the 128-column tile and all BM rows).
template <int FMT, int BM, int EPI, int ST>
__global__ __launch_bounds__(256) void op_gemm_ring_kernel(OpGemmArgs a) {
  static_assert(FMT != 2 && ST >= 2 && ST <= 8 && BM >= 16 && BM <= 64 && (EPI != OP_LMH || BM == 16), "ring GEMM shape");
  using R = OpRing<FMT, BM>;
  const OpHdr hd = op_hdr(a.c);
#define OP_RING_ARR(i) __shared__ __attribute__((aligned(16))) uint4 r##i[ST > i ? R::N : 1];
  OP_RING_ARR(0) OP_RING_ARR(1) OP_RING_ARR(2) OP_RING_ARR(3) OP_RING_ARR(4) OP_RING_ARR(5) OP_RING_ARR(6) OP_RING_ARR(7)
#undef OP_RING_ARR
  __shared__ uint64_t red[4][16];   // (the argmax epilogue only)
  auto ring = [&](int d) -> uint4* {
    return d == 0 ? r0 : d == 1 ? r1 : d == 2 ? r2 : d == 3 ? r3 : d == 4 ? r4 : d == 5 ? r5 : d == 6 ? r6 : r7;
  };
  constexpr int TM = BM / 16;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  // (tiles renumbered per XCD for the 32- and 64-row prefill tiles but gate/up, as
  // op_gemm_kernel; the argmax epilogue indexes by blockIdx.x)
  const OpTile tl = EPI != OP_SILU && BM > 16 ? op_tile_xcd() : OpTile{(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z};
  const int n0 = tl.x * OP_BN, m0 = tl.y * BM;
  const int K = a.W.K, qg = a.W.qg;
  const int kb = tl.z * a.ksteps * OP_BK;
  const int ns = (min(K, kb + a.ksteps * OP_BK) - kb) / OP_BK;
  v4f acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; i++) {
    acc[i][0] = (v4f){0.f, 0.f, 0.f, 0.f};
    acc[i][1] = (v4f){0.f, 0.f, 0.f, 0.f};
  }
  // QKV: the epilogue's bias values and rotary rows (at the expected positions pos_hint +
  // row), loaded while the k-steps stream (loaded in the epilogue they cost a memory round
  // trip each, about 4 us per workgroup)
  float2 qcs[EPI == OP_QKV ? TM * 4 : 1];
  float qbias[2];
  if constexpr (EPI == OP_QKV) {
    const int b = (n0 + 32 * w) >> 5;
    const float* bq = a.c.L[a.layer].bqkv + 32 * b + n;
    qbias[0] = gld(bq);
    qbias[1] = gld(bq + 16);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        qcs[4 * i + r] = gld(a.c.rope + (size_t)min(a.pos_hint + m0 + 16 * i + 4 * kg + r, a.c.maxctx - 1) * 32 + (b & 1) * 16 + n);
  }
  // steps past the slice reload its last one, so that every stage issues the same loads
#pragma unroll
  for (int d = 0; d < ST - 1; d++) op_ring_load<FMT, BM>(a, m0, n0, kb + min(d, ns - 1) * OP_BK, ring(d), tid);
  int s0 = 0;
  for (; s0 + ST <= ns; s0 += ST) {
#pragma unroll
    for (int d = 0; d < ST; d++) {
      op_ring_wait<R::L>(ST - 2);
      op_ring_load<FMT, BM>(a, m0, n0, kb + min(s0 + d + ST - 1, ns - 1) * OP_BK, ring((d + ST - 1) % ST), tid);
      op_ring_mma<FMT, BM>(ring(d), w, kg, n, qg, acc);
    }
  }
#pragma unroll
  for (int d = 0; d < ST - 1; d++)
    if (s0 + d < ns) {
      op_ring_wait<R::L>(ST - 2 - d);
      op_ring_mma<FMT, BM>(ring(d), w, kg, n, qg, acc);
    }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no LDS load outlives the workgroup
  if constexpr (EPI == OP_QKV) op_gemm_epilogue<BM, EPI>(a, hd, acc, m0, n0, tl.z, w, kg, n, red, a.pos_hint, qcs, qbias);
  else op_gemm_epilogue<BM, EPI>(a, hd, acc, m0, n0, tl.z, w, kg, n, red);
}

// ---- GEMM of passes of up to 16 rows --------------------------------------------------
// Workgroup: 4 waves, wave w owns columns n0 + 32 w .. + 31 (two 16-column MFMA tiles) and
// rows 0-15. The A rows of the K slice sit in LDS for the whole kernel (filled once, one
// barrier); each wave loads its own weight operands straight into registers (no LDS, no
// barrier in the k loop), OP_SDEPTH(FMT) k-steps of them in flight. Within a k-step lane (kg, n)
// takes columns 16 kg .. 16 kg + 15 of the 64 (8 for each of the two MFMAs), a permutation
// of k applied to A and W alike. With SILU the A operand is the SwiGLU unit
// f16(silu(g) * u) of the gate/up GEMM's K-slice partials (summed in slice order, as
// op_epi_kernel does), so that no separate SiLU kernel runs. The host uses it for that
// down projection only: for the other small-pass GEMMs the LDS-tiled op_gemm_kernel<.., 16,
// ..> measured as fast (q8) or faster (f16: about 3 us per step-kernel).
#define OP_SDEPTH(FMT) ((FMT) == 0 ? 4 : 8)   // f16 k-steps carry twice the bytes of q8 ones
#define OP_SMAXK 1024   // K slice columns at most (16 k-steps)

template <int FMT>
struct BOp {   // one k-step's weights of one lane for the wave's two column tiles
  uint4 q[2][FMT == 0 ? 2 : 1];   // q4: .x .y hold the 16 nibbles
  // q8: scale (kept 16-bit: widening the loaded value would wait for it at once);
  // q4: (scale, min)
  std::conditional_t<FMT == 2, uint32_t, uint16_t> s[2];
};
template <int FMT>
__device__ __forceinline__ void op_fetch_b(const OpMat& W, int col0, int k0, int kg, int n, BOp<FMT>& b) {
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const size_t row = (size_t)(col0 + 16 * j + n);
    const int k = k0 + 16 * kg;
    if constexpr (FMT == 2) {
      const uint2 v = gld((const uint2*)(W.w + row * (W.K / 2) + k / 2));
      b.q[j][0] = make_uint4(v.x, v.y, 0u, 0u);
      b.s[j] = gld((const uint32_t*)(W.s + (row * (W.K / 64) + k / 64) * 2));
    } else if constexpr (FMT == 1) {
      b.q[j][0] = gld((const uint4*)(W.w + op_wt_off((int)row, k, W.K, 1)));
      b.s[j] = gld(W.s + op_st_off((int)row, k, W.K, W.qg));
    } else {
      b.q[j][0] = gld((const uint4*)(W.w + op_wt_off((int)row, k, W.K, 2)));
      b.q[j][1] = gld((const uint4*)(W.w + op_wt_off((int)row, k + 8, W.K, 2)));
    }
  }
}
// the 8 f16 operand values of MFMA half ks (k = 16 kg + 8 ks ..) of column tile j
template <int FMT>
__device__ __forceinline__ v8h op_bvals(const BOp<FMT>& b, int j, int ks) {
  v8h o;
  if constexpr (FMT == 2) {
    const _Float16 sc = (_Float16)h2f(b.s[j] & 0xffff), mn = (_Float16)h2f(b.s[j] >> 16);
    const uint32_t x = ks == 0 ? b.q[j][0].x : b.q[j][0].y;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t byte = (x >> (8 * i)) & 0xff;
      o[2 * i] = sc * (_Float16)(float)(byte & 15) + mn;
      o[2 * i + 1] = sc * (_Float16)(float)(byte >> 4) + mn;
    }
  } else if constexpr (FMT == 1) {
    const _Float16 sc = (_Float16)h2f(b.s[j]);
    const uint32_t x0 = ks == 0 ? b.q[j][0].x : b.q[j][0].z, x1 = ks == 0 ? b.q[j][0].y : b.q[j][0].w;
    _Float16 h[8];
    op_q8x4(x0, sc, h);
    op_q8x4(x1, sc, h + 4);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = h[i];
  } else {
    o = u4_to_v8h(b.q[j][ks]);
  }
  return o;
}

template <int FMT, int EPI, bool SILU, int NWV = 4>
__global__ __launch_bounds__(64 * NWV) void op_gemv_kernel(OpGemmArgs a) {
  // NWV 4: four waves, 32 columns each. NWV 2 (the unsplit QKV GEMM): two waves share 32
  // columns and split the K steps in halves, added (wave 0's + wave 1's) before the
  // epilogue, which wave 0 applies.
  static_assert(NWV == 4 || (NWV == 2 && EPI == OP_QKV), "two-wave workgroups: the unsplit QKV GEMM");
  constexpr bool KS2 = NWV == 2;
  constexpr int NT = 64 * NWV;
  const OpHdr hd = op_hdr(a.c);
  __shared__ __attribute__((aligned(16))) _Float16 As[16 * (OP_SMAXK + 8)];
  __shared__ uint64_t red[4][16];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int n0 = blockIdx.x * (KS2 ? 32 : 32 * NWV), col0 = n0 + (KS2 ? 0 : 32 * w);
  // QKV: the rotary rows of this lane's rows 4 kg + r at the expected position (pos_hint + row)
  float2 cs[4];
  if constexpr (EPI == OP_QKV) {
#pragma unroll
    for (int r = 0; r < 4; r++)
      cs[r] = gld(a.c.rope + (size_t)min(a.pos_hint + 4 * kg + r, a.c.maxctx - 1) * 32 + ((col0 >> 5) & 1) * 16 + n);
  }
  const int K = a.W.K;
  const int kb = blockIdx.z * a.ksteps * OP_BK, ke = min(K, kb + a.ksteps * OP_BK);
  const int nsa = (ke - kb) / OP_BK, kw = ke - kb;
  const int lda = kw + 8;   // LDS row stride (halves)
  // this wave's k-steps: all of the slice, or (KS2) its half
  const int s_lo = KS2 ? w * nsa / NWV : 0;
  const int ns = KS2 ? (w + 1) * nsa / NWV - s_lo : nsa;
  const int kbw = kb + s_lo * OP_BK;   // the wave's first column
  constexpr int SD = OP_SDEPTH(FMT);
  BOp<FMT> ring[SD];
#pragma unroll
  for (int d = 0; d < SD; d++) {
    op_fetch_b<FMT>(a.W, col0, kbw + min(d, ns - 1) * OP_BK, kg, n, ring[d]);
    __builtin_amdgcn_sched_barrier(0);   // issue order = slot order (the waits count on it)
  }
  // A rows 0 .. M-1 of the slice into LDS (rows >= M are left as they are: their outputs
  // are never stored)
  if constexpr (!SILU) {
    const int per = kw / 8;   // uint4 per row
    for (int i = tid; i < a.M * per; i += NT) {
      const int m = i / per, c8 = i - m * per;
      *(uint4*)(As + m * lda + 8 * c8) = gld((const uint4*)(a.A + (size_t)m * K + kb) + c8);
    }
  } else {
    // units kb + 2 p, kb + 2 p + 1 of row m: gate/up columns 2 kb + 4 p .. + 3 (g, g, u, u)
    const int per = kw / 2, N2 = 2 * K;
    for (int i = tid; i < a.M * per; i += NT) {
      const int m = i / per, p = i - m * per;
      float4 pz[OP_MAXS];
#pragma unroll
      for (int z = 0; z < OP_MAXS; z++)
        if (z < a.aS) pz[z] = gld((const float4*)(a.apart + ((size_t)z * a.M + m) * N2 + 2 * kb) + p);
      float4 v = pz[0];
#pragma unroll
      for (int z = 1; z < OP_MAXS; z++)
        if (z < a.aS) {
          v.x += pz[z].x;
          v.y += pz[z].y;
          v.z += pz[z].z;
          v.w += pz[z].w;
        }
      As[m * lda + 2 * p] = (_Float16)__float2half(v.x / (1.0f + expf(-v.x)) * v.z);
      As[m * lda + 2 * p + 1] = (_Float16)__float2half(v.y / (1.0f + expf(-v.y)) * v.w);
    }
  }
  __syncthreads();
  v4f acc[1][2];
  acc[0][0] = (v4f){0.f, 0.f, 0.f, 0.f};
  acc[0][1] = (v4f){0.f, 0.f, 0.f, 0.f};
  auto kstep = [&](int d, int st, bool refetch) {
    v8h bf[2][2];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int ks = 0; ks < 2; ks++) bf[j][ks] = op_bvals<FMT>(ring[d], j, ks);
    if (refetch) {
      __builtin_amdgcn_sched_barrier(0);
      op_fetch_b<FMT>(a.W, col0, kbw + min(st + SD, ns - 1) * OP_BK, kg, n, ring[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const v8h af = *(const v8h*)(As + n * lda + (s_lo + st) * OP_BK + 16 * kg + 8 * ks);
#pragma unroll
      for (int j = 0; j < 2; j++) acc[0][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j][ks], acc[0][j], 0, 0, 0);
    }
  };
  int s0 = 0;
  for (; s0 + SD <= ns; s0 += SD) {
#pragma unroll
    for (int d = 0; d < SD; d++) kstep(d, s0 + d, true);
  }
#pragma unroll
  for (int d = 0; d < SD - 1; d++)
    if (s0 + d < ns) kstep(d, s0 + d, false);
  if constexpr (KS2) {
    __shared__ v4f kacc[NWV][2][64];
    if (w > 0) {
      kacc[w][0][lane] = acc[0][0];
      kacc[w][1][lane] = acc[0][1];
    }
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int ww = 1; ww < NWV; ww++)
#pragma unroll
      for (int jj = 0; jj < 2; jj++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[0][jj][r] = acc[0][jj][r] + kacc[ww][jj][lane][r];
    op_gemm_epilogue<16, EPI>(a, hd, acc, 0, n0, (int)blockIdx.z, 0, kg, n, red, a.pos_hint, cs);
  } else {
    op_gemm_epilogue<16, EPI>(a, hd, acc, 0, n0, (int)blockIdx.z, w, kg, n, red, a.pos_hint, cs);
  }
}

// Split-K reduction: sum of the slices' partials in slice order, then the epilogue.
// RESID / SILU / QKV: one thread per output column / unit / rotary pair of a row.
template <int EPI>
__global__ __launch_bounds__(256) void op_epi_kernel(OpGemmArgs a, int S) {
  const OpHdr hd = op_hdr(a.c);
  const int N = a.W.N;
  const int per = EPI == OP_RESID ? N : N / 2;   // SILU: units; QKV: pairs
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= a.M * per) return;
  const int m = i / per, j = i % per;
  // every slice's partial in flight at once, then added in slice order
  auto sum = [&](int col) {
    float pz[OP_MAXS];
#pragma unroll
    for (int z = 0; z < OP_MAXS; z++) pz[z] = z < S ? gld(a.part + ((size_t)z * a.M + m) * N + col) : 0.f;
    float v = pz[0];
#pragma unroll
    for (int z = 1; z < OP_MAXS; z++)
      if (z < S) v += pz[z];
    return v;
  };
  if constexpr (EPI == OP_RESID) {
    float* r = a.resid + (size_t)m * ILL_H + j;
    const float x = gld(r), y = sum(j);
    if (!hd.done) gst(r, x + y);
  } else if constexpr (EPI == OP_SILU) {
    const int q = j >> 1, r = j & 1;
    const float g = sum(4 * q + r), u = sum(4 * q + 2 + r);
    if (!hd.done) epi_silu(a.c, m, j, g, u);
  } else if constexpr (EPI == OP_QKV) {
    const int b = j >> 4, ii = j & 15;
    const int at = min(a.pos_hint + m, a.c.maxctx - 1);   // a chain row's expected position
    const float2 cs = gld(a.c.rope + (size_t)at * 32 + (b & 1) * 16 + ii);
    const float x0 = sum(32 * b + ii), x1 = sum(32 * b + 16 + ii);
    if (!hd.done) epi_qkv(a.c, hd, a.layer, m, b, ii, x0, x1, at, cs);
  }
}

// Residual split-K reduction fused with the RMSNorm that reads the updated residual, for
// passes of up to 16 rows: one workgroup per row m, one thread per column. x[m] += the
// slices' partials (added in slice order, as op_epi_kernel); then, for rows m >= row0,
// xn[m - row0] = f16(x * rsqrt(mean(x^2) + eps) * gamma), the sum of squares taken per wave
// and the 14 wave sums added in order (a function of the row alone, so 1-row and 16-row
// passes agree bit for bit).
__global__ __launch_bounds__(ILL_H) void op_epi_norm_kernel(OpGemmArgs a, int S, const float* gamma, int row0) {
  __shared__ float red[ILL_H / 64];
  const OpHdr hd = op_hdr(a.c);
  const int m = blockIdx.x, j = threadIdx.x, w = j >> 6, lane = j & 63;
  float pz[OP_MAXS];
#pragma unroll
  for (int z = 0; z < OP_MAXS; z++) pz[z] = z < S ? gld(a.part + ((size_t)z * a.M + m) * ILL_H + j) : 0.f;
  float* r = a.resid + (size_t)m * ILL_H + j;
  const float g = gld(gamma + j);
  float y = pz[0];
#pragma unroll
  for (int z = 1; z < OP_MAXS; z++)
    if (z < S) y += pz[z];
  const float v = gld(r) + y;
  if (!hd.done) gst(r, v);
  if (m < row0) return;   // the whole workgroup
  const float ss = gsum<64>(v * v);
  if (lane == 0) red[w] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < ILL_H / 64; i++) tot += red[i];
  const float scale = __builtin_amdgcn_rsqf(tot * (1.0f / (float)ILL_H) + ILL_EPS);
  if (hd.done) return;
  gst((uint16_t*)(a.c.xn + (size_t)(m - row0) * ILL_H + j), (uint16_t)__half_as_ushort(__float2half(v * scale * g)));
}

// ---- attention of passes of up to 16 rows -------------------------------------------------
// Row t attends to virtual positions 0 .. L-1, L = pos + depth(t) + 1; position p lives in
// cache slot p below pos and in slot pos + (the row on t's path at depth p - pos) above
// (tree passes; chains use slot p). The row's 64-position chunks are dealt to 64 slots:
// chunk c to slot (split s = (c / 16) % 8, wave w = c % 8), so a context of up to 1024
// positions is all split 0. Slot (s, w) folds its chunks in increasing order with the pass
// kernel's rule, the eight slots of split s are combined against their maximum (in w
// order), then the eight splits against theirs (in s order).
// The grouping depends only on the row's L, not on M or on how the work is launched, so a
// row decoded alone and the same row inside a 16-row pass give identical bits.
// One workgroup of 8 waves per (row t, query head h, part j < nsplit) runs the splits j,
// j + nsplit, ...: with nsplit = 1 it finishes the row; otherwise it stores its split
// states and op_attn_combine_kernel finishes the row. (The host picks nsplit from the
// context length it expects; any value gives the same result.)
#define OP_NSPLIT 8
#define OP_SPLIT_W 66   // scratch words per split state: m, l, o[64]
#define OP_VST 72       // LDS stride (halves) of a staged V row

// (m, l, o) of n states combined against their maximum, in index order; states with
// m = -inf (no positions) add nothing, and if all are empty the result is empty too.
template <int N>
__device__ __forceinline__ void att_combine(const float* m, const float* l, const float* o, float& mo, float& lo, float& oo) {
  float mm = m[0];
#pragma unroll
  for (int i = 1; i < N; i++) mm = fmaxf(mm, m[i]);
  float sum = 0.f, acc = 0.f;
  if (mm != -INFINITY) {
#pragma unroll
    for (int i = 0; i < N; i++) {
      const float e = att_exp(m[i] - mm);
      sum = sum + l[i] * e;
      acc = acc + o[i] * e;
    }
  }
  mo = mm;
  lo = sum;
  oo = acc;
}

// The O projection of one (row, head) folded into the attention kernel (passes of up to 16
// rows, one attention split): wave w computes output columns 112 w + lane and
// 112 w + 64 + lane (lane < 48) of W_o[:, 64 h .. 64 h + 63] . ao, where ao is the head's
// f16 output (LDS). Weights are dequantized as op_gemm_kernel does (q8: f16 s * q; f16 as
// stored) and the 64 products are added in k order in fp32: the partial of slice h, which
// op_epi_norm_kernel sums over the 14 heads in head order.
template <int FMT>
struct ORows {
  uint4 q[2][FMT == 0 ? 8 : 4];
  uint32_t s[2];   // q8: the scales of k 0-31 (low half) and 32-63 (high; equal for group 64)
};
// Woh: the head-major copy (OpLayerW::oh), so each load reads 1 KB contiguous over the lanes
template <int FMT>
__device__ __forceinline__ void orows_fetch(const OpMat& Woh, int h, int w, int lane, ORows<FMT>& o) {
  constexpr int NC = FMT == 0 ? 8 : 4;   // 16-byte chunks of a row's 64 columns
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = min(112 * w + 64 * u + lane, ILL_H - 1);
    const uint4* src = (const uint4*)Woh.w + (size_t)h * NC * ILL_H + r;
#pragma unroll
    for (int i = 0; i < NC; i++) o.q[u][i] = gld(src + (size_t)i * ILL_H);
    if constexpr (FMT == 1) o.s[u] = gld((const uint32_t*)Woh.s + (size_t)h * ILL_H + r);
  }
}
template <int FMT>
__device__ __forceinline__ void orows_apply(const ORows<FMT>& o, const _Float16* ao, int w, int lane, float* dst) {
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int r = 112 * w + 64 * u + lane;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < (FMT == 0 ? 8 : 4); i++) {
      const uint32_t x[4] = {o.q[u][i].x, o.q[u][i].y, o.q[u][i].z, o.q[u][i].w};
      constexpr int PER = FMT == 0 ? 8 : 16;   // k values per uint4
      _Float16 wq[FMT == 1 ? 16 : 1];
      if constexpr (FMT == 1) {   // k = 16 i + e: the scale of k / 32 = i / 2
        const _Float16 sc = (_Float16)h2f((uint16_t)(o.s[u] >> (16 * (i >> 1))));
#pragma unroll
        for (int q = 0; q < 4; q++) op_q8x4(x[q], sc, wq + 4 * q);
      }
#pragma unroll
      for (int e = 0; e < PER; e++) {
        const int k = PER * i + e;
        _Float16 wv;
        if constexpr (FMT == 1) wv = wq[e];
        else wv = __ushort_as_half((unsigned short)((x[e >> 1] >> (16 * (e & 1))) & 0xffff));
        acc = fmaf((float)wv, (float)ao[k], acc);
      }
    }
    if (u == 0 || lane < 48) dst[r] = acc;
  }
}

template <int FMT>
__global__ __launch_bounds__(64 * ILL_WAVES) void op_attn_kernel(OpCtx c, int layer, int M, int nsplit, float* scratch,
                                                               OpMat Wo, float* opart) {
  __shared__ __attribute__((aligned(16))) float qs[ILL_WAVES][64];   // a copy per wave
  __shared__ __attribute__((aligned(16))) float ps[ILL_WAVES][64];
  __shared__ int path[16];
  __shared__ float cm[OP_NSPLIT][ILL_WAVES], cl[OP_NSPLIT][ILL_WAVES], co[OP_NSPLIT][ILL_WAVES][64];
  __shared__ float sm[OP_NSPLIT], sl[OP_NSPLIT], so[OP_NSPLIT][64];
  __shared__ __attribute__((aligned(16))) uint16_t vstage[ILL_WAVES][64 * OP_VST];   // tree passes: V rows
  __shared__ _Float16 aoh[64];   // with opart: the head's output, the O projection's input
  const OpHdr hd = op_hdr(c);
  constexpr bool SWZ = FMT != 2;   // the cache layout of the q8 / f16 engines (ill_common.h)
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rh = blockIdx.x / nsplit, j = blockIdx.x % nsplit;
  const int t = rh / ILL_NH, h = rh % ILL_NH, g = h / 7;
  const float qv = gld(c.q + (size_t)t * ILL_H + h * 64 + lane);   // before the K/V loads
  // with opart (nsplit 1, q8 / f16) the O projection follows (this wave's W_o rows are
  // fetched when the chunk loop is done: held from the start they would spill)
  constexpr bool OFUSE = FMT != 2;
  const bool fused = OFUSE && opart != nullptr;
  ORows<OFUSE ? FMT : 1> orw;
  const uint16_t* kb = c.kc + ((size_t)layer * ILL_NKV + g) * c.maxctx * 64;
  const uint16_t* vb = c.vt + ((size_t)layer * ILL_NKV + g) * (c.maxctx / 64) * 4096;
  // The wave's first chunk (split j, chunk 16 j + w) at its plain slots, issued before the
  // header is waited for; it is used unless the chunk lies past the row's positions or
  // holds pass rows of a tree pass (their slots come from the path table).
  uint4 kv[8], vv[8];
  const int ch0 = 16 * j + w;
  {
    const int ks = min(64 * ch0 + lane, c.maxctx - 1), vc = min(ch0, c.maxctx / 64 - 1);
#pragma unroll
    for (int i = 0; i < 8; i++) kv[i] = gld((const uint4*)(kb + kv_k_off(ks, 8 * i, SWZ)));
#pragma unroll
    for (int i = 0; i < 8; i++) vv[i] = gld((const uint4*)(vb + kv_v_off(64 * vc + 8 * i, lane, SWZ)));
  }
  const int pos = hd.pos;
  const bool tree = hd.mode == ILL_MODE_TREE;
  const int dep = op_depth(c, hd.mode, t);
  const int L = pos + dep + 1;
  const int nch = (L + 63) >> 6;
  const int nne = min(OP_NSPLIT, (nch + 15) >> 4);   // splits 0 .. nne - 1 hold chunks
  // chunk ch: the K row of position 64 ch + lane (slot remapped along the path in tree
  // passes) and the V values of dim = lane
  auto fetch = [&](int ch, uint4 (&kv)[8], uint4 (&vv)[8]) {
    const int vp = 64 * ch + lane;
    const int slot = min(vp < pos || !tree ? vp : pos + path[min(max(vp - pos, 0), 15)], c.maxctx - 1);
#pragma unroll
    for (int i = 0; i < 8; i++) kv[i] = gld((const uint4*)(kb + kv_k_off(slot, 8 * i, SWZ)));
#pragma unroll
    for (int i = 0; i < 8; i++) vv[i] = gld((const uint4*)(vb + kv_v_off(64 * ch + 8 * i, lane, SWZ)));
  };
  const bool early = j < nne && ch0 < nch && (!tree || 64 * ch0 + 63 < pos);
  qs[w][lane] = qv * 0.125f;
  if (w == 0 && lane < 16) {   // rows on t's path by depth (tree passes: depth <= 15)
    int pr = lane;
    if (tree) {
      int r = t;
      for (int d = dep; d >= 0; --d) {
        if (d == lane) pr = r;
        r = r > 0 ? gld(c.tree + ILL_TR_PARENT + r) : 0;
      }
    }
    path[lane] = pr;
  }
  lds_barrier();   // path and qs visible; the chunk loads stay in flight
#pragma unroll 1
  for (int q = 0; q < OP_NSPLIT; q++) {
    const int s = j + nsplit * q;
    if (s >= nne) break;
    float Mx = -INFINITY, Ls = 0.f, O = 0.f;
    // this wave's chunks of split s: 128 r + 16 s + 8 b + w (r = 0, 1, ..., b = 0, 1) in
    // order; the next one streams in while one is evaluated
    auto chunk_of = [&](int i) { return 128 * (i >> 1) + 16 * s + 8 * (i & 1) + w; };
    int ch = chunk_of(0);
    if (ch < nch && !(q == 0 && early)) fetch(ch, kv, vv);
    for (int ci = 0; ch < nch; ch = chunk_of(++ci)) {
      uint4 kn[8], vn[8];
      const int nx = chunk_of(ci + 1);
      const bool more = nx < nch;
      if (more) fetch(nx, kn, vn);
      const int vp = 64 * ch + lane;
      const bool valid = vp < L;
      float sc = 0.f;
      // q is re-read from LDS for every chunk (broadcast reads): held in registers it would
      // push the two K/V buffers out of them
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t x[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
        const float4 qa = *(const float4*)&qs[w][8 * i], qb = *(const float4*)&qs[w][8 * i + 4];
        const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int e = 0; e < 8; e++) sc = fmaf(qv[e], h2f(x[e >> 1] >> (16 * (e & 1))), sc);
      }
      sc = valid ? sc : -INFINITY;
      const float mc = gmax<64>(sc);
      const float p = valid ? att_exp(sc - mc) : 0.f;
      const float lc = gsum<64>(p);
      ps[w][lane] = p;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      float oc = 0.f;
      if (tree && 64 * ch + 63 >= pos) {   // wave-uniform: positions pos .. L-1 of the chunk
        // take the V of the path rows' slots: this lane's V row goes through LDS, where
        // those (at most 16) positions are replaced
        uint16_t* vr = &vstage[w][lane * OP_VST];
#pragma unroll
        for (int i = 0; i < 8; i++) *(uint4*)(vr + 8 * i) = vv[i];
        const int p0 = max(pos - 64 * ch, 0), p1 = min(L - 64 * ch, 64);
        uint16_t pv[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
          const int pp = p0 + k;
          if (pp < p1) {
            const int sl2 = pos + path[64 * ch + pp - pos];
            pv[k] = gld(vb + kv_v_off(sl2, lane, SWZ));
          }
        }
#pragma unroll
        for (int k = 0; k < 16; k++)
          if (p0 + k < p1) vr[p0 + k] = pv[k];
#pragma unroll
        for (int i = 0; i < 8; i++) vv[i] = *(const uint4*)(vr + 8 * i);
      }
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t x[4] = {vv[i].x, vv[i].y, vv[i].z, vv[i].w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int pp = 8 * i + e, vq = 64 * ch + pp;
          float v = h2f(x[e >> 1] >> (16 * (e & 1)));
          v = vq < L ? v : 0.f;
          oc = fmaf(ps[w][pp], v, oc);
        }
      }
      __builtin_amdgcn_wave_barrier();
      const AttScale k = att_scale(Mx, mc);
      O = att_fold(O, oc, k);
      Ls = att_fold(Ls, lc, k);
      Mx = k.mn;
      if (more) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
          kv[i] = kn[i];
          vv[i] = vn[i];
        }
      }
    }
    if (lane == 0) {
      cm[q][w] = Mx;
      cl[q][w] = Ls;
    }
    co[q][w][lane] = O;
  }
  if constexpr (OFUSE)
    if (fused) orows_fetch<FMT>(Wo, h, w, lane, orw);
  __syncthreads();
  // the head's output row: to c.ao, or (opart) through LDS into the O projection
  auto emit = [&](float v) {
    const __half hv = __float2half(v);
    if (fused) aoh[lane] = (_Float16)hv;
    else if (!hd.done) gst((uint16_t*)(c.ao + (size_t)t * ILL_H + h * 64 + lane), (uint16_t)__half_as_ushort(hv));
  };
  auto oproj = [&]() {
    if constexpr (OFUSE) {
      __syncthreads();
      orows_apply<FMT>(orw, aoh, w, lane, opart + ((size_t)h * M + t) * ILL_H);
    }
  };
  if (nsplit == 1 && nne == 1) {   // one split: its state is the row's (the general path
    if (w == 0) {                  // below gives the same bits: scale 1, nothing added)
      float o[ILL_WAVES];
#pragma unroll
      for (int ww = 0; ww < ILL_WAVES; ww++) o[ww] = co[0][ww][lane];
      float mo, lo, oo;
      att_combine<ILL_WAVES>(cm[0], cl[0], o, mo, lo, oo);
      emit(oo / lo);
    }
    if (fused) oproj();
    return;
  }
  // split states: wave q combines the slots of split j + nsplit q (empty splits: m = -inf)
  const int nq = (OP_NSPLIT - j + nsplit - 1) / nsplit;
  if (w < nq) {
    if (j + nsplit * w >= nne) {   // no chunks: nothing was stored for it
      if (lane == 0) {
        cm[w][0] = -INFINITY;
        cl[w][0] = 0.f;
      }
#pragma unroll
      for (int ww = 1; ww < ILL_WAVES; ww++)
        if (lane == 0) cm[w][ww] = -INFINITY;
    }
    float o[ILL_WAVES];
#pragma unroll
    for (int ww = 0; ww < ILL_WAVES; ww++) o[ww] = co[w][ww][lane];
    float mo, lo, oo;
    att_combine<ILL_WAVES>(cm[w], cl[w], o, mo, lo, oo);
    if (nsplit == 1) {
      if (lane == 0) {
        sm[w] = mo;
        sl[w] = lo;
      }
      so[w][lane] = oo;
    } else {
      float* dst = scratch + ((size_t)rh * OP_NSPLIT + j + nsplit * w) * OP_SPLIT_W;
      if (lane == 0) {
        dst[0] = mo;
        dst[1] = lo;
      }
      dst[2 + lane] = oo;
    }
  }
  if (nsplit > 1) return;
  __syncthreads();
  if (w == 0) {
    float o[OP_NSPLIT];
#pragma unroll
    for (int q = 0; q < OP_NSPLIT; q++) o[q] = so[q][lane];
    float mo, lo, oo;
    att_combine<OP_NSPLIT>(sm, sl, o, mo, lo, oo);
    emit(oo / lo);
  }
  if (fused) oproj();
}

// The rows of op_attn_kernel launched with nsplit > 1: the eight split states of (row, head)
// combined in split order (wave 0), then (opart) the head's O projection by all eight waves.
template <int FMT>
__global__ __launch_bounds__(64 * ILL_WAVES) void op_attn_combine_kernel(OpCtx c, const float* scratch, OpMat Wo, float* opart,
                                                                       int M) {
  __shared__ _Float16 aoh[64];
  const int done = gld(&c.st->done);
  const int rh = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = rh / ILL_NH, h = rh % ILL_NH;
  // with opart (q8 / f16) the head's O projection follows, as in op_attn_kernel
  constexpr bool OFUSE = FMT != 2;
  const bool fused = OFUSE && opart != nullptr;
  ORows<OFUSE ? FMT : 1> orw;
  if constexpr (OFUSE)
    if (fused) orows_fetch<FMT>(Wo, h, w, lane, orw);
  if (w == 0) {
    float m[OP_NSPLIT], l[OP_NSPLIT], o[OP_NSPLIT];
#pragma unroll
    for (int s = 0; s < OP_NSPLIT; s++) {
      const float* src = scratch + ((size_t)rh * OP_NSPLIT + s) * OP_SPLIT_W;
      m[s] = gld(src);
      l[s] = gld(src + 1);
      o[s] = gld(src + 2 + lane);
    }
    float mo, lo, oo;
    att_combine<OP_NSPLIT>(m, l, o, mo, lo, oo);
    const __half hv = __float2half(oo / lo);
    if (fused) aoh[lane] = (_Float16)hv;
    else if (!done) gst((uint16_t*)(c.ao + (size_t)t * ILL_H + h * 64 + lane), (uint16_t)__half_as_ushort(hv));
  }
  if constexpr (OFUSE)
    if (fused) {
      __syncthreads();
      orows_apply<FMT>(orw, aoh, w, lane, opart + ((size_t)h * M + t) * ILL_H);
    }
}

// ---- attention of prefill chunks (more than 16 rows): MFMA flash attention --------------
// One workgroup of OP_RW waves per (16-row block, query head h): chunk c goes to wave
// c % OP_RW, which folds its chunks in order, and the waves' states are combined at the end
// in wave order. Row t < M sits at position pos + t and attends to positions 0 .. pos + t,
// all in the cache (this chunk's QKV kernel has written its own keys and values). Per
// 64-position chunk: scores (0.125 q) . k on v_mfma_f32_16x16x32_f16 with q split into f16
// high and low parts (products as accurate as fp32 q), the causal mask, the row softmax statistics (maximum, sum of exponentials) folded chunk by chunk with
// the rule of the other attention kernels, and O += P V with P split the same way. A wave's
// next chunk's keys and values stream in while one is evaluated.
#define OP_RW 4
// P round trip through LDS: rows of 68 floats, so that the row-strided writes (4 kg + j)
// and the per-lane row reads (n) spread over the 64 banks (rows of 64 put a wave's 16 row
// reads, and its 4 kg groups' writes, on the same banks)
#define OP_PLD 68
template <bool SWZ>   // the K/V cache layout (ill_common.h): swizzled for q8 / f16, rows for q4
__global__ __launch_bounds__(64 * OP_RW) void op_attn_rows_kernel(OpCtx c, int layer, int M) {
  __shared__ __attribute__((aligned(16))) float pbw[OP_RW][16 * OP_PLD];
  __shared__ float sm_[OP_RW][16], sl_[OP_RW][16], so_[OP_RW][16][64];
  const OpHdr hd = op_hdr(c);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, kg = lane >> 4, n = lane & 15;
  float* pb = pbw[w];
  const int t0 = 16 * blockIdx.x, h = blockIdx.y, g = h / 7;
  const int pos = hd.pos;
  // A operand: lane (kg, n) holds row t0 + n, dims 32 ks + 8 kg + i
  v8h qa[2][2];
  {
    const float* qr = c.q + (size_t)min(t0 + n, M - 1) * ILL_H + h * 64;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const uint4 a0 = gld((const uint4*)(qr + 32 * ks + 8 * kg)), a1 = gld((const uint4*)(qr + 32 * ks + 8 * kg + 4));
      const uint32_t x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float v = __uint_as_float(x[i]) * 0.125f;
        const _Float16 hi = (_Float16)v;
        qa[ks][0][i] = hi;
        qa[ks][1][i] = (_Float16)(v - (float)hi);
      }
    }
  }
  int Lr[4];   // L of this lane's rows t0 + 4 kg + j (0: no row)
#pragma unroll
  for (int j = 0; j < 4; j++) Lr[j] = t0 + 4 * kg + j < M ? pos + t0 + 4 * kg + j + 1 : 0;
  const int nch = (pos + min(t0 + 16, M) + 63) >> 6;
  const uint16_t* kbase = c.kc + ((size_t)layer * ILL_NKV + g) * c.maxctx * 64;
  const uint16_t* vbase = c.vt + ((size_t)layer * ILL_NKV + g) * (c.maxctx / 64) * 64 * 64;
  float Mx[4], Ls[4], O[4][4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    Mx[j] = -INFINITY;
    Ls[j] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; nb++) O[nb][j] = 0.f;
  }
  KVFrag f;
  if (w < nch) kv_fetch<SWZ>(kbase, vbase, w, lane, f);
  for (int ch = w; ch < nch; ch += OP_RW) {
    KVFrag fn;
    const bool more = ch + OP_RW < nch;
    if (more) kv_fetch<SWZ>(kbase, vbase, ch + OP_RW, lane, fn);
    float sc[4][4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
      v4f sv = {0.f, 0.f, 0.f, 0.f};
      sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][0], u4_to_v8h(f.k[b][0]), sv, 0, 0, 0);
      sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][1], u4_to_v8h(f.k[b][0]), sv, 0, 0, 0);
      sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][0], u4_to_v8h(f.k[b][1]), sv, 0, 0, 0);
      sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][1], u4_to_v8h(f.k[b][1]), sv, 0, 0, 0);
      const int vp = 64 * ch + 16 * b + n;
#pragma unroll
      for (int j = 0; j < 4; j++) sc[b][j] = vp < Lr[j] ? sv[j] : -INFINITY;
    }
    float mx[4], ls[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      mx[j] = gmax<16>(fmaxf(fmaxf(sc[0][j], sc[1][j]), fmaxf(sc[2][j], sc[3][j])));
      const float ms = mx[j] == -INFINITY ? 0.f : mx[j];   // a row with no position here: p = 0
      float sum = 0.f;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        sc[b][j] = att_exp(sc[b][j] - ms);
        sum += sc[b][j];
      }
      ls[j] = gsum<16>(sum);
#pragma unroll
      for (int b = 0; b < 4; b++) pb[(4 * kg + j) * OP_PLD + 16 * b + n] = sc[b][j];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    v8h ph[2], pl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float p = pb[n * OP_PLD + 32 * ks + 8 * kg + i];
        const _Float16 hi = (_Float16)p;
        ph[ks][i] = hi;
        pl[ks][i] = (_Float16)(p - (float)hi);
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[0], u4_to_v8h(f.v[nb][0]), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[0], u4_to_v8h(f.v[nb][0]), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[1], u4_to_v8h(f.v[nb][1]), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[1], u4_to_v8h(f.v[nb][1]), acc, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if (mx[j] == -INFINITY) continue;   // nothing of this row in the chunk
        const AttScale k = att_scale(Mx[j], mx[j]);
        O[nb][j] = att_fold(O[nb][j], acc[j], k);
        if (nb == 3) {
          Ls[j] = att_fold(Ls[j], ls[j], k);
          Mx[j] = k.mn;
        }
      }
    }
    if (more) f = fn;
  }
  // the waves' states, combined in wave order against their maximum
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (n == 0) {
      sm_[w][4 * kg + j] = Mx[j];
      sl_[w][4 * kg + j] = Ls[j];
    }
#pragma unroll
    for (int nb = 0; nb < 4; nb++) so_[w][4 * kg + j][16 * nb + n] = O[nb][j];
  }
  __syncthreads();
  if (hd.done) return;
  const int r = threadIdx.x >> 4, t = t0 + r;
  if (t >= M) return;
  float m[OP_RW], l[OP_RW];
#pragma unroll
  for (int i = 0; i < OP_RW; i++) {
    m[i] = sm_[i][r];
    l[i] = sl_[i][r];
  }
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int d = (threadIdx.x & 15) + 16 * q;
    float o[OP_RW];
#pragma unroll
    for (int i = 0; i < OP_RW; i++) o[i] = so_[i][r][d];
    float mo, lo, oo;
    att_combine<OP_RW>(m, l, o, mo, lo, oo);
    gst((uint16_t*)(c.ao + (size_t)t * ILL_H + h * 64 + d), (uint16_t)__half_as_ushort(__float2half(oo / lo)));
  }
}

// ---- commit ----------------------------------------------------------------------------
// Global argmax of rows lmh0 .. lmh0 + lmhn - 1 over the lm_head tiles, then the same
// commit as the pass kernel (greedy, chain or tree accept, KV compaction, State advance).
__global__ __launch_bounds__(ILL_WG_THREADS) void op_commit_kernel(IllPassArgs a, const uint64_t* amax, int ntiles, int kvswz) {
  __shared__ PassHdr H;
  __shared__ CommitLds C;
  __shared__ uint64_t best[ILL_WAVES];
  load_hdr(a, H);
  if (H.done) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  int stopreq = 0;   // the host's stop word (see ill_pass_kernel), waited for at the commit
  if (tid == 0 && a.stop_host) stopreq = __hip_atomic_load((const GAS int32_t*)a.stop_host, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  for (int t = H.lmh0; t < H.lmh0 + H.lmhn; t++) {
    uint64_t k = 0;
    for (int i = tid; i < ntiles; i += ILL_WG_THREADS) {
      const uint64_t kk = amax[(size_t)i * 16 + t];
      k = kk > k ? kk : k;
    }
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t ok = __shfl_xor(k, o, 64);
      k = ok > k ? ok : k;
    }
    if (lane == 0) best[w] = k;
    __syncthreads();
    if (tid == 0) {
      uint64_t m = best[0];
      for (int i = 1; i < ILL_WAVES; i++) m = best[i] > m ? best[i] : m;
      C.g[t] = (int)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFu));
    }
    __syncthreads();
  }
  commit_apply(a, H, C, false, stopreq, kvswz != 0);
}
