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
  const uint8_t* w;    // q4: codes [N][K/2]; q8: int8 [N][K]; f16: [N][K]
  const uint16_t* s;   // q4: [N][K/64][2] f16 (scale, min); q8: [N][K/qg] f16; f16: unused
  int N, K, qg;        // qg: q8 group size (32 or 64)
};

struct OpLayerW {
  OpMat qkv, o, gu, d;
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
};

// Row t's position offset from pos (its depth): tree passes read the tree, others are chains.
__device__ __forceinline__ int op_depth(const OpCtx& c, int t) {
  return c.ctl->mode == ILL_MODE_TREE ? c.tree[ILL_TR_DEPTH + t] : (c.ctl->mode == ILL_MODE_DECODE ? 0 : t);
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
    const float q = (float)(int8_t)m.w[(size_t)r * m.K + k];
    return h2f(m.s[(size_t)r * (m.K / m.qg) + k / m.qg]) * q;
  } else {
    return h2f(((const uint16_t*)m.w)[(size_t)r * m.K + k]);
  }
}

// x[t][:] = embedding row of ptoks[t] (Shaders.swift:118-126, :179-190)
template <int FMT>
__global__ __launch_bounds__(256) void op_embed_kernel(OpCtx c, int M) {
  if (c.st->done) return;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= M * ILL_H) return;
  const int t = i / ILL_H, k = i % ILL_H;
  c.x[i] = op_dequant1<FMT>(c.emb, c.ptoks[t], k);
}

// xn[t] = f16(x[t] * rsqrt(mean(x^2) + eps) * gamma) for rows row0 .. row0 + M - 1 (one wave
// per row; sum of squares in a fixed order). Output row index t - row0.
__global__ __launch_bounds__(256) void op_norm_kernel(OpCtx c, const float* gamma, int row0, int M) {
  if (c.st->done) return;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + w;
  if (t >= M) return;
  const float* xr = c.x + (size_t)(row0 + t) * ILL_H;
  float v[14];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 14; i++) {
    v[i] = xr[64 * i + lane];
    ss += v[i] * v[i];
  }
  ss = gsum<64>(ss);
  const float scale = __builtin_amdgcn_rsqf(ss * (1.0f / (float)ILL_H) + ILL_EPS);
#pragma unroll
  for (int i = 0; i < 14; i++) c.xn[(size_t)t * ILL_H + 64 * i + lane] = __float2half(v[i] * scale * gamma[64 * i + lane]);
}

// ---- GEMM: Y[M][N] = A[M][K] (f16) * W[N][K]^T, fused epilogues ------------------------
enum OpEpi { OP_QKV = 0, OP_RESID = 1, OP_SILU = 2, OP_LMH = 3 };

struct OpGemmArgs {
  OpCtx c;
  const __half* A;   // [M][K]
  OpMat W;
  int M, layer;
  float* resid;      // OP_RESID: [M][896] += Y
};

#define OP_BN 128
#define OP_BK 64
#define OP_LDK 72    // LDS row stride in halves (padding against bank conflicts)

// Dequantize W rows n0 .. n0+127, columns k0 .. k0+63 into LDS [128][OP_LDK] f16.
template <int FMT>
__device__ __forceinline__ void op_load_w(const OpMat& W, int n0, int k0, _Float16* Bs, int tid) {
  if constexpr (FMT == 2) {
    // 128 rows x 32 bytes: thread -> (row, 16-byte half)
    const int r = tid >> 1, hf = tid & 1;
    const uint4 b = gld((const uint4*)(W.w + (size_t)(n0 + r) * (W.K / 2) + k0 / 2 + 16 * hf));
    const uint32_t sm = gld((const uint32_t*)(W.s + ((size_t)(n0 + r) * (W.K / 64) + k0 / 64) * 2));
    const _Float16 s = (_Float16)h2f(sm & 0xffff), m = (_Float16)h2f(sm >> 16);
    const uint32_t x[4] = {b.x, b.y, b.z, b.w};
    _Float16 o[32];
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t byte = (x[i >> 2] >> (8 * (i & 3))) & 0xff;
      o[2 * i] = s * (_Float16)(float)(byte & 15) + m;
      o[2 * i + 1] = s * (_Float16)(float)(byte >> 4) + m;
    }
    _Float16* dst = Bs + r * OP_LDK + 32 * hf;
#pragma unroll
    for (int i = 0; i < 4; i++) *(uint4*)(dst + 8 * i) = *(const uint4*)(o + 8 * i);
  } else if constexpr (FMT == 1) {
    // 128 rows x 64 bytes: thread -> (row, 32-byte half)
    const int r = tid >> 1, hf = tid & 1;
    const uint8_t* src = W.w + (size_t)(n0 + r) * W.K + k0 + 32 * hf;
    const uint4 b0 = gld((const uint4*)src), b1 = gld((const uint4*)(src + 16));
    const int kk = k0 + 32 * hf;
    const _Float16 s = (_Float16)h2f(gld(W.s + (size_t)(n0 + r) * (W.K / W.qg) + kk / W.qg));
    const uint32_t x[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    _Float16 o[32];
#pragma unroll
    for (int i = 0; i < 32; i++) o[i] = s * (_Float16)(float)(int8_t)((x[i >> 2] >> (8 * (i & 3))) & 0xff);
    _Float16* dst = Bs + r * OP_LDK + 32 * hf;
#pragma unroll
    for (int i = 0; i < 4; i++) *(uint4*)(dst + 8 * i) = *(const uint4*)(o + 8 * i);
  } else {
    // 128 rows x 128 bytes: thread -> (row, 64-byte half)
    const int r = tid >> 1, hf = tid & 1;
    const uint4* src = (const uint4*)(W.w + ((size_t)(n0 + r) * W.K + k0 + 32 * hf) * 2);
    _Float16* dst = Bs + r * OP_LDK + 32 * hf;
#pragma unroll
    for (int i = 0; i < 4; i++) *(uint4*)(dst + 8 * i) = gld(src + i);
  }
}

// Workgroup: 256 threads = 4 waves; a wave owns 32 columns (two 16-column MFMA tiles) of
// the 128-column tile and all BM rows.
template <int FMT, int BM, int EPI>
__global__ __launch_bounds__(256) void op_gemm_kernel(OpGemmArgs a) {
  if (a.c.st->done) return;
  __shared__ __attribute__((aligned(16))) _Float16 As[BM * OP_LDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[OP_BN * OP_LDK];
  __shared__ uint64_t red[4][16];
  constexpr int TM = BM / 16;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int n0 = blockIdx.x * OP_BN, m0 = blockIdx.y * BM;
  const int K = a.W.K;
  v4f acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; i++) {
    acc[i][0] = (v4f){0.f, 0.f, 0.f, 0.f};
    acc[i][1] = (v4f){0.f, 0.f, 0.f, 0.f};
  }
  for (int k0 = 0; k0 < K; k0 += OP_BK) {
    // A: BM rows x 64 halves (rows >= M read row M-1: finite, and their outputs are unused)
    for (int i = tid; i < BM * 8; i += 256) {
      const int r = i >> 3, ch = i & 7;
      const int mr = min(m0 + r, a.M - 1);
      *(uint4*)(As + r * OP_LDK + 8 * ch) = gld((const uint4*)(a.A + (size_t)mr * K + k0) + ch);
    }
    op_load_w<FMT>(a.W, n0, k0, Bs, tid);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      v8h bf[2];
#pragma unroll
      for (int j = 0; j < 2; j++) bf[j] = *(const v8h*)(Bs + (32 * w + 16 * j + n) * OP_LDK + 32 * ks + 8 * kg);
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const v8h af = *(const v8h*)(As + (16 * i + n) * OP_LDK + 32 * ks + 8 * kg);
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // ---- epilogues: lane holds rows 16 i + 4 kg + r, columns n0 + 32 w + 16 j + n
  const OpCtx& c = a.c;
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
    // gate/up rows in groups of 4: g[2q], g[2q+1], u[2q], u[2q+1] (Convert.swift:134-136)
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float v = acc[i][j][r];
          const float up = __shfl_down(v, 2, 16);
          const int m = m0 + 16 * i + 4 * kg + r, col = n0 + 32 * w + 16 * j + n;
          if ((n & 3) < 2 && m < a.M) {
            const int unit = (col >> 2) * 2 + (n & 3);
            c.h[(size_t)m * ILL_FF + unit] = __float2half(v / (1.0f + expf(-v)) * up);
          }
        }
  } else if constexpr (EPI == OP_QKV) {
    // a wave's 32 columns are one rotary block b: tile 0 = dims d, tile 1 = dims d + 32
    // (Convert.swift:236-244); head b/2: q heads 0-13, k 14-15, v 16-17
    const int b = (n0 + 32 * w) >> 5, head = b >> 1;
    const int d = (b & 1) * 16 + n;
    const float b0 = c.L[a.layer].bqkv[32 * b + n], b1 = c.L[a.layer].bqkv[32 * b + 16 + n];
    const int pos = c.st->pos;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + 16 * i + 4 * kg + r;
        if (m >= a.M) continue;
        float x0 = acc[i][0][r] + b0, x1 = acc[i][1][r] + b1;
        if (head < ILL_NH + ILL_NKV) {
          const float2 cs = c.rope[(pos + op_depth(c, m)) * 32 + d];
          const float r0 = x0 * cs.x - x1 * cs.y, r1 = x1 * cs.x + x0 * cs.y;
          x0 = r0;
          x1 = r1;
        }
        const int slot = pos + m;
        if (head < ILL_NH) {
          c.q[(size_t)m * ILL_H + head * 64 + d] = x0;
          c.q[(size_t)m * ILL_H + head * 64 + d + 32] = x1;
        } else if (head < ILL_NH + ILL_NKV) {
          uint16_t* kr = c.kc + (((size_t)a.layer * ILL_NKV + (head - ILL_NH)) * c.maxctx + slot) * 64;
          kr[d] = (uint16_t)f2h(x0);
          kr[d + 32] = (uint16_t)f2h(x1);
        } else {
          uint16_t* vb = c.vt + (((size_t)a.layer * ILL_NKV + (head - ILL_NH - ILL_NKV)) * (c.maxctx / 64) + slot / 64) * 4096;
          vb[d * 64 + (slot & 63)] = (uint16_t)f2h(x0);
          vb[(d + 32) * 64 + (slot & 63)] = (uint16_t)f2h(x1);
        }
      }
  } else {   // OP_LMH: logits (optional) and per-tile argmax keys per row (BM == 16)
    const int wlog = c.ctl->write_logits;
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

// ---- attention: one wave per (row, query head) --------------------------------------
// Row t attends to virtual positions 0 .. L-1, L = pos + depth(t) + 1; position p lives
// in cache slot p below pos and in slot pos + (the row on t's path at depth p - pos) above
// (tree passes; chains use slot p). Chunks of 64 positions in order, each folded into the
// running (max, sum, output) with the same rule as the pass kernel.
__global__ __launch_bounds__(256) void op_attn_kernel(OpCtx c, int layer, int M) {
  if (c.st->done) return;
  __shared__ float qs[4][64];
  __shared__ float ps[4][64];
  __shared__ int path[4][16];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + w;
  if (pair >= M * ILL_NH) return;
  const int t = pair / ILL_NH, h = pair % ILL_NH, g = h / 7;
  const int pos = c.st->pos;
  const bool tree = c.ctl->mode == ILL_MODE_TREE;
  const int dep = op_depth(c, t);
  const int L = pos + dep + 1;
  if (lane < 16) {   // rows on t's path by depth (tree passes)
    int r = t, pr = 0;
    for (int d = dep; d >= 0; --d) {
      if (d == lane) pr = r;
      r = r > 0 && tree ? c.tree[ILL_TR_PARENT + r] : r - 1;
    }
    path[w][lane] = tree ? pr : lane;
  }
  qs[w][lane] = c.q[(size_t)t * ILL_H + h * 64 + lane] * 0.125f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const uint16_t* kb = c.kc + ((size_t)layer * ILL_NKV + g) * c.maxctx * 64;
  const uint16_t* vb = c.vt + ((size_t)layer * ILL_NKV + g) * (c.maxctx / 64) * 4096;
  float Mx = -INFINITY, Ls = 0.f, O = 0.f;
  const int nch = (L + 63) >> 6;
  for (int ch = 0; ch < nch; ch++) {
    const int vp = 64 * ch + lane;
    const bool valid = vp < L;
    const int slot = min(vp < pos || !tree ? vp : pos + path[w][min(vp - pos, 15)], c.maxctx - 1);
    // score of position vp (lane = position)
    const uint4* kr = (const uint4*)(kb + (size_t)slot * 64);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint4 u = gld(kr + i);
      const uint32_t x[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 8; e++) s = fmaf(qs[w][8 * i + e], h2f(x[e >> 1] >> (16 * (e & 1))), s);
    }
    s = valid ? s : -INFINITY;
    const float mc = gmax<64>(s);
    const float p = valid ? att_exp(s - mc) : 0.f;
    const float lc = gsum<64>(p);
    ps[w][lane] = p;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // P.V for dim = lane over the chunk's 64 positions (transposed V: 64 slots per row)
    const uint4* vr = (const uint4*)(vb + ((size_t)ch * 64 + lane) * 64);
    float oc = 0.f;
    const bool remap = tree && 64 * ch + 63 >= pos;   // wave-uniform
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint4 u = gld(vr + i);
      const uint32_t x[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int pp = 8 * i + e, vq = 64 * ch + pp;
        float v = h2f(x[e >> 1] >> (16 * (e & 1)));
        if (remap && vq >= pos && vq < L) {
          const int sl = pos + path[w][vq - pos];
          v = h2f(vb[((size_t)(sl >> 6) * 64 + lane) * 64 + (sl & 63)]);
        }
        v = vq < L ? v : 0.f;
        oc = fmaf(ps[w][pp], v, oc);
      }
    }
    __builtin_amdgcn_wave_barrier();
    const AttScale k = att_scale(Mx, mc);
    O = att_fold(O, oc, k);
    Ls = att_fold(Ls, lc, k);
    Mx = k.mn;
  }
  c.ao[(size_t)t * ILL_H + h * 64 + lane] = __float2half(O / Ls);
}

// ---- commit ----------------------------------------------------------------------------
// Global argmax of rows lmh0 .. lmh0 + lmhn - 1 over the lm_head tiles, then the same
// commit as the pass kernel (greedy, chain or tree accept, KV compaction, State advance).
__global__ __launch_bounds__(ILL_WG_THREADS) void op_commit_kernel(IllPassArgs a, const uint64_t* amax, int ntiles) {
  __shared__ PassHdr H;
  __shared__ CommitLds C;
  __shared__ uint64_t best[ILL_WAVES];
  if (threadIdx.x == 0) load_hdr(a, H);
  __syncthreads();
  if (H.done) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
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
  commit_apply(a, H, C, false);
}
