// Device helpers of the MI355X decode engine: tagged words, bounded waits, MFMA tiles.
//
// Within one pass kernel, every value that crosses workgroups is a 64-bit word
// (payload | tag << 32) written and read with agent-scope atomics. Agent-scope atomics are
// coherent across the eight XCD L2s, so no cache writeback/invalidate fence is needed,
// and a consumer waits for exactly the words it reads (no grid barrier). The tag is
// epoch * 32 + layer + 1; the epoch advances once per pass, so a word from an earlier
// pass or layer never passes the check.
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include "ill_common.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

#define ILL_WAIT_TICKS 200000000ull   // 2 s of the 100 MHz constant clock

// Every device-side access to HBM goes through these helpers, which name the global
// address space explicitly. Pointers taken from the argument struct are otherwise generic
// and compile to FLAT instructions, which also count against lgkmcnt: every later LDS read
// would then wait for all outstanding HBM loads and atomics of the wave.
#define GAS __attribute__((address_space(1)))
typedef unsigned int gu32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int gu32x2 __attribute__((ext_vector_type(2)));
template <class T>
__device__ __forceinline__ T gld(const T* p) {
  T r;
  if constexpr (sizeof(T) == 16) {
    const gu32x4 x = *(const GAS gu32x4*)p;
    __builtin_memcpy(&r, &x, 16);
  } else if constexpr (sizeof(T) == 8) {
    const gu32x2 x = *(const GAS gu32x2*)p;
    __builtin_memcpy(&r, &x, 8);
  } else {
    r = *(const GAS T*)p;
  }
  return r;
}
template <class T>
__device__ __forceinline__ void gst(T* p, T v) { *(GAS T*)p = v; }

__device__ __forceinline__ uint64_t aload64(const uint64_t* p) {
  return __hip_atomic_load((const GAS uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void astore64(uint64_t* p, uint64_t v) {
  __hip_atomic_store((GAS uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t aload32(const int32_t* p) {
  return __hip_atomic_load((const GAS int32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void astore32(int32_t* p, int32_t v) {
  __hip_atomic_store((GAS int32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t mkw(float v, uint32_t tag) {
  return ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}
__device__ __forceinline__ uint64_t mkwu(uint32_t v, uint32_t tag) { return ((uint64_t)tag << 32) | (uint64_t)v; }
__device__ __forceinline__ bool wok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float wval(uint64_t w) { return __uint_as_float((uint32_t)w); }

__device__ __forceinline__ uint64_t clk() { return wall_clock64(); }

// Tag of the lm_head argmax partials of a pass.
__device__ __forceinline__ uint32_t tagof_lmh(uint32_t epoch) { return epoch * 32u + 31u; }

// Records the first timeout code; every wait gives up once any is recorded.
__device__ __forceinline__ void set_err(IllCtl* ctl, int code) {
  int32_t zero = 0;
  __hip_atomic_compare_exchange_strong((GAS int32_t*)&ctl->err, &zero, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup-wide bounded wait: `ready()` is evaluated by every thread (it loads the words
// the thread needs and checks their tags). Returns false (uniformly) on timeout or when
// another workgroup has already recorded an error.
// The error flag and the clock are consulted every 32nd poll only, so a wait that succeeds
// early costs one memory round trip per poll and nothing else.
template <class F>
__device__ __forceinline__ bool wg_wait(F&& ready, IllCtl* ctl, int code) {
  const uint64_t t0 = clk();
  for (int it = 1;; it++) {
    const bool ok = ready();
    if (__syncthreads_and(ok)) return true;
    if ((it & 31) == 0) {
      int bad = 0;
      if (threadIdx.x == 0) {
        bad = aload32(&ctl->err) != 0;
        if (!bad && clk() - t0 > ILL_WAIT_TICKS) { set_err(ctl, code); bad = 1; }
      }
      if (__syncthreads_or(bad)) return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Wave-wide bounded wait (lanes of one wave only). On failure the caller must still reach
// the next workgroup barrier and report its failure there.
template <class F>
__device__ __forceinline__ bool wave_wait(F&& ready, IllCtl* ctl, int code) {
  const uint64_t t0 = clk();
  for (int it = 1;; it++) {
    const bool ok = ready();
    if (__all(ok)) return true;
    if ((it & 31) == 0) {
      if (aload32(&ctl->err) != 0) return false;
      if (clk() - t0 > ILL_WAIT_TICKS) { set_err(ctl, code); return false; }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Two-stage wave-wide bounded wait: polls `light()` (a word or two per row, loaded by every
// lane from one address, so one memory request each) until it holds, then `ready()` (the
// whole input) as wave_wait does. The input completes as a whole, so the light words turn
// ready with it, and a wave that waits long costs a request per row per poll instead of
// its whole input's. `ready()` alone decides success.
template <class L, class F>
__device__ __forceinline__ bool wave_wait2(L&& light, F&& ready, IllCtl* ctl, int code) {
  const uint64_t t0 = clk();
  bool lit = false;
  for (int it = 1;; it++) {
    if (!lit) lit = __all(light());
    if (lit && __all(ready())) return true;
    if ((it & 31) == 0) {
      if (aload32(&ctl->err) != 0) return false;
      if (clk() - t0 > ILL_WAIT_TICKS) { set_err(ctl, code); return false; }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// The light stage of wave_wait2 alone, pipelined: D polls of the light words in flight, each
// iteration checks the oldest and issues it again (samples every round trip / D). `issue(st)`
// loads the light words into st, `check(st)` tests them. False on an error or a timeout.
// (SLEEP: s_sleep units of 64 cycles between iterations.)
template <int D, int SLEEP, class W, class I, class C>
__device__ __forceinline__ bool wave_light_p(I&& issue, C&& check, IllCtl* ctl, int code) {
  const uint64_t t0 = clk();
  W st[D];
#pragma unroll
  for (int d = 0; d < D; d++) issue(st[d]);
  for (int it = 1;; it++) {
    bool lit = false;
#pragma unroll
    for (int d = 0; d < D; d++)
      if (!lit) {
        lit = __all(check(st[d]));
        if (!lit) issue(st[d]);
      }
    if (lit) return true;
    if constexpr (SLEEP > 0) __builtin_amdgcn_s_sleep(SLEEP);
    if ((it & 7) == 0) {
      if (aload32(&ctl->err) != 0) return false;
      if (clk() - t0 > ILL_WAIT_TICKS) { set_err(ctl, code); return false; }
    }
  }
}

// A wave-uniform value held in a vector register, so that loads from addresses built on it
// stay vector memory loads.
__device__ __forceinline__ int vgpr_uniform(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ bool wg_failed(IllCtl* ctl) {
  int bad = 0;
  if (threadIdx.x == 0) bad = aload32(&ctl->err) != 0;
  return __syncthreads_or(bad);
}

// ---- wave reductions ---------------------------------------------------------------------
// Reductions over aligned lane groups of 2^k lanes with cross-lane moves that stay out of
// LDS: DPP quad permutes (partners l^1, l^2), row half-mirror and row mirror (partners
// within 8 and 16 lanes), then permlane16/32 swaps (the other row / the other half-wave).
// Every stage combines a lane's value with one partner's and both partners compute the
// same commutative operation, so every lane of the group ends with the same value, and
// the association order is fixed.
#define ILL_DPP_XOR1 0xB1    // quad_perm [1,0,3,2]
#define ILL_DPP_XOR2 0x4E    // quad_perm [2,3,0,1]
#define ILL_DPP_HMIR 0x141   // row_half_mirror
#define ILL_DPP_MIR 0x140    // row_mirror
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }

// Combine over groups of N lanes (N = 2, 4, ..., 64) with operation `op`.
template <int N, class V, class Op>
__device__ __forceinline__ V group_reduce(V v, Op op) {
  auto dpp = [](V x, auto ctrl_tag) {
    constexpr int C = decltype(ctrl_tag)::value;
    if constexpr (sizeof(V) == 4 && __is_same(V, float)) return dpp_f<C>(x);
    else return (V)dpp_i<C>((int)x);
  };
  v = op(v, dpp(v, std::integral_constant<int, ILL_DPP_XOR1>{}));
  if constexpr (N >= 4) v = op(v, dpp(v, std::integral_constant<int, ILL_DPP_XOR2>{}));
  if constexpr (N >= 8) v = op(v, dpp(v, std::integral_constant<int, ILL_DPP_HMIR>{}));
  if constexpr (N >= 16) v = op(v, dpp(v, std::integral_constant<int, ILL_DPP_MIR>{}));
  if constexpr (N >= 32) {
    int bits;
    __builtin_memcpy(&bits, &v, 4);
    const auto r = __builtin_amdgcn_permlane16_swap(bits, bits, false, false);
    V a, b;
    const int r0 = (int)r[0], r1 = (int)r[1];
    __builtin_memcpy(&a, &r0, 4);
    __builtin_memcpy(&b, &r1, 4);
    v = op(a, b);
  }
  if constexpr (N >= 64) {
    int bits;
    __builtin_memcpy(&bits, &v, 4);
    const auto r = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
    V a, b;
    const int r0 = (int)r[0], r1 = (int)r[1];
    __builtin_memcpy(&a, &r0, 4);
    __builtin_memcpy(&b, &r1, 4);
    v = op(a, b);
  }
  return v;
}
struct OpAddF { __device__ float operator()(float a, float b) const { return a + b; } };
struct OpMaxF { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpAddI { __device__ int operator()(int a, int b) const { return a + b; } };
struct OpMaxU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };
template <int N> __device__ __forceinline__ float gsum(float v) { return group_reduce<N>(v, OpAddF{}); }
template <int N> __device__ __forceinline__ float gmax(float v) { return group_reduce<N>(v, OpMaxF{}); }
template <int N> __device__ __forceinline__ int gsumi(int v) { return group_reduce<N>(v, OpAddI{}); }
// max |v| over the group, as an integer maximum of the magnitudes' bit patterns (ordered
// like the values for non-negative floats)
template <int N> __device__ __forceinline__ float gmaxabs(float v) {
  return __uint_as_float(group_reduce<N>(__float_as_uint(v) & 0x7fffffffu, OpMaxU{}));
}

// Order-preserving 64-bit key of (value, index): larger value first, then lower index.
__device__ __forceinline__ uint64_t amax_key(float v, int idx) {
  const uint32_t b = __float_as_uint(v + 0.0f);   // -0 orders as +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)bits16));
}
__device__ __forceinline__ uint32_t f2h(float v) { return (uint32_t)__half_as_ushort(__float2half_rn(v)); }
// f16 with saturation to the finite range (NaN to the largest finite value): what the V
// cache stores, so that every V slot holds a finite value and a zero probability times an
// unused slot is zero
__device__ __forceinline__ uint32_t f2h_sat(float v) { return f2h(__builtin_amdgcn_fmed3f(v, -65504.0f, 65504.0f)); }

// ---- activation quantization ------------------------------------------------------------
// A row of activations is coded per 64-column group as 16-bit fixed point
// v = rint(x / d), d = max|x| / 32639, split into int8 hi = (v + 128) >> 8 and
// lo = v - 256 hi, so an int8 MFMA over hi and lo gives sum(w*v) exactly.
// Byte p of a lane's 16-byte operand holds column 16*kg + kPerm[p]: the order in which
// a 4-bit weight word unpacks (low nibbles of 4 bytes, then high nibbles).
__device__ __forceinline__ int q4perm(int p) {
  // 0,2,4,6, 1,3,5,7, 8,10,12,14, 9,11,13,15
  return ((p >> 3) << 3) | ((p & 3) << 1) | ((p >> 2) & 1);
}
#define ILL_QMAX 32639.0f

// 16 values (cols 16*kg + i, i = 0..15) of one row -> operand bytes (q4 order), local sums.
__device__ __forceinline__ void quant16(const float* v, float d, uint32_t hi[4], uint32_t lo[4], int& sumq) {
  int q[16];
  sumq = 0;
  const float inv = d > 0.f ? __builtin_amdgcn_rcpf(d) : 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    q[i] = (int)rintf(v[i] * inv);
    sumq += q[i];
  }
#pragma unroll
  for (int r = 0; r < 4; r++) { hi[r] = 0; lo[r] = 0; }
#pragma unroll
  for (int p = 0; p < 16; p++) {
    const int x = q[q4perm(p)];
    const int h = (x + 128) >> 8;
    const int l = x - (h << 8);
    hi[p >> 2] |= ((uint32_t)(h & 0xff)) << (8 * (p & 3));
    lo[p >> 2] |= ((uint32_t)(l & 0xff)) << (8 * (p & 3));
  }
}

// ---- q4 tile machinery ----------------------------------------------------------------
// A repacked q4 row tile (16 rows x 896 columns) is 7 blocks of 1 KiB; in block cb, lane
// l = 16*kg + n holds 16 bytes: row n, columns 128*cb + 16*kg .. +16 (bytes 0-7, group 2cb)
// and 128*cb + 64 + 16*kg .. +16 (bytes 8-15, group 2cb+1), two columns per byte (even
// column in the low nibble). Scales: 7 x 128 B; lane n reads (scale, min) f16 pairs of
// row n for both groups.
struct Q4Tile {
  uint4 w[ILL_KST];
  uint2 s[ILL_KST];
};

__device__ __forceinline__ void q4_load(Q4Tile& t, const uint8_t* wtile, const uint32_t* stile, int lane) {
  const int n = lane & 15;
#pragma unroll
  for (int cb = 0; cb < ILL_KST; cb++) {
    t.w[cb] = gld((const uint4*)(wtile + cb * 1024 + lane * 16));
    t.s[cb] = gld((const uint2*)(stile + cb * 32 + n * 2));
  }
}

// Asynchronous HBM -> LDS copy of `bytes` (a multiple of 16) by one wave: each lane moves 16 B
// per instruction with global_load_lds_dwordx4 (no registers involved). Completion is
// tracked by the wave's vmcnt; the LDS destination must be 16-byte aligned.
__device__ __forceinline__ void wave_copy_to_lds(const uint8_t* src, uint8_t* lds_dst, int bytes, int lane) {
  for (int off = 0; off < bytes; off += 1024) {
    const int rem = bytes - off;
    if (lane * 16 < rem)
      __builtin_amdgcn_global_load_lds((const void*)(src + off + lane * 16),
                                       (__attribute__((address_space(3))) void*)(lds_dst + off), 16, 0, 0);
  }
}
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0); }

__device__ __forceinline__ v4i q4_unpack(uint32_t a, uint32_t b) {
  v4i r;
  r[0] = (int)(a & 0x0F0F0F0Fu);
  r[1] = (int)((a >> 4) & 0x0F0F0F0Fu);
  r[2] = (int)(b & 0x0F0F0F0Fu);
  r[3] = (int)((b >> 4) & 0x0F0F0F0Fu);
  return r;
}

// Prepared activations of a K = 896 input in LDS (see prep896): A operands per group G,
// lane-group kg and row m, and per (G, row) the pair (d, X = d * sum(v)).
template <int T>
struct PrepLds {
  uint4 ahi[14 * 4 * T];
  uint4 alo[14 * 4 * T];
  float2 sc[14 * T];          // per (group, row): step d and d * sum of the codes
  alignas(16) float red[ILL_WAVES][T];   // per-wave partial sums of squares
  alignas(16) int ok[ILL_WAVES];         // per-wave "input complete" votes
  int lit;                               // 1-row passes: the watcher wave's verdict
};

// MFMA A-operand row read by lane row m: at T = 1 every lane row aliases row 0, so the
// tile's 16 output rows are copies of row 0 and no lane reads outside the T rows held.
template <int T>
__device__ __forceinline__ int arow(int m) { return T == 1 ? 0 : (m & (T - 1)); }

// Opaque copy of a per-lane value: address arithmetic derived from it is redone at each use
// instead of being hoisted out of enclosing loops into long-lived registers.
__device__ __forceinline__ int opq(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// A operand of group G for this lane at T = 1: the tile's 16 output rows need one input
// row, so lane rows m = 0 and 1 carry its high and low bytes and one MFMA gives both
// products (D row 0 = hi . W, row 1 = lo . W: the same integers as two MFMAs would).
template <int T>
__device__ __forceinline__ const uint4* t1_abase(const PrepLds<T>& P, int lane) {
  return (lane & 1) ? P.alo : P.ahi;
}

// Accumulate 16-row tiles over K = 896: acc[i][j] (rows t = 4*kg + j of the pass, weight
// row n of tile i) += sum_G s*d*S + m*X. The per-value operation sequence is independent
// of T and of NT. `fetch(i, cb, w, s)` supplies tile i's block cb: 16 weight bytes and the
// (scale, min) pairs for this lane. The body has no branches, so the compiler can issue
// every operand read before the first MFMA; rows >= nrows produce values that callers
// ignore. With NT > 1 the tiles share each group's A-operand and (d, X) reads (LDS reads,
// not MFMAs, bound these tiles) and their MFMA chains interleave.
template <int T, int NT, class Fetch>
__device__ __forceinline__ void q4_tiles896f(Fetch fetch, const PrepLds<T>& P, int lane_, float (*acc)[4]) {
  static_assert(NT == 1 || NT == 2, "one or two interleaved tiles");
  const int lane = opq(lane_);
  const int kg = lane >> 4, m = arow<T>(lane & 15);
  constexpr int RPL = T >= 4 ? 4 : T;
  uint4 wv[NT][ILL_KST];
  uint2 sv[NT][ILL_KST];
#pragma unroll
  for (int i = 0; i < NT; i++) {
#pragma unroll
    for (int cb = 0; cb < ILL_KST; cb++) fetch(i, cb, wv[i][cb], sv[i][cb]);
  }
  const v4i z = {0, 0, 0, 0};
  // T = 1: every A operand is read before the first MFMA (the group chain would otherwise
  // wait for each read in turn)
  uint4 xa[T == 1 ? 2 * ILL_KST : 1];
  if (T == 1) {
    const uint4* a1 = t1_abase<T>(P, lane);
#pragma unroll
    for (int G = 0; G < 2 * ILL_KST; G++) xa[G] = a1[G * 4 + kg];
    __builtin_amdgcn_sched_barrier(0);
  }
  // T = 1: every group's MFMA is issued before the group epilogues (which run in group
  // order), so the products stream through the matrix pipe instead of each one's latency
  // being waited for in the accumulation chain
  int S1[T == 1 ? NT : 1][T == 1 ? 2 * ILL_KST : 1];
  if (T == 1) {
#pragma unroll
    for (int G = 0; G < 2 * ILL_KST; G++) {
      const int cb = G >> 1, gi = G & 1;
      const uint4 x = xa[G];
      const v4i ax = (v4i){(int)x.x, (int)x.y, (int)x.z, (int)x.w};
#pragma unroll
      for (int i = 0; i < NT; i++) {
        const v4i b = gi == 0 ? q4_unpack(wv[i][cb].x, wv[i][cb].y) : q4_unpack(wv[i][cb].z, wv[i][cb].w);
        const v4i dd = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, b, z, 0, 0, 0);
        S1[i][G] = (dd[0] << 8) + dd[1];
      }
    }
  }
#pragma unroll
  for (int G = 0; G < 2 * ILL_KST; G++) {
    const int cb = G >> 1, gi = G & 1;
    if (T == 1) {
      const float2 dx = P.sc[G];
#pragma unroll
      for (int i = 0; i < NT; i++) {
        const uint32_t sm = gi == 0 ? sv[i][cb].x : sv[i][cb].y;
        const float sw = h2f(sm & 0xffff), mw = h2f(sm >> 16);
        const float t1 = dx.x * (float)S1[i][G];
        acc[i][0] = fmaf(sw, t1, acc[i][0]);
        acc[i][0] = fmaf(mw, dx.y, acc[i][0]);
      }
    } else {
      const uint4 h = P.ahi[(G * 4 + kg) * T + m];
      const uint4 l = P.alo[(G * 4 + kg) * T + m];
      const v4i ah = (v4i){(int)h.x, (int)h.y, (int)h.z, (int)h.w};
      const v4i al = (v4i){(int)l.x, (int)l.y, (int)l.z, (int)l.w};
      float2 dx[RPL];
#pragma unroll
      for (int j = 0; j < RPL; j++) dx[j] = P.sc[G * T + arow<T>(4 * kg + j)];
#pragma unroll
      for (int i = 0; i < NT; i++) {
        const v4i b = gi == 0 ? q4_unpack(wv[i][cb].x, wv[i][cb].y) : q4_unpack(wv[i][cb].z, wv[i][cb].w);
        const v4i dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, b, z, 0, 0, 0);
        const v4i dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, b, z, 0, 0, 0);
        const uint32_t sm = gi == 0 ? sv[i][cb].x : sv[i][cb].y;
        const float sw = h2f(sm & 0xffff), mw = h2f(sm >> 16);
#pragma unroll
        for (int j = 0; j < RPL; j++) {
          const int S = (dh[j] << 8) + dl[j];
          const float t1 = dx[j].x * (float)S;
          acc[i][j] = fmaf(sw, t1, acc[i][j]);
          acc[i][j] = fmaf(mw, dx[j].y, acc[i][j]);
        }
      }
      // At T > 1 each group needs 4 rows of (d, X): pin each group's epilogue to its group
      // and bound the scheduler's read-ahead to two groups, so the operands and MFMA
      // results of a whole tile are not held in registers at once.
#pragma unroll
      for (int i = 0; i < NT; i++) {
#pragma unroll
        for (int j = 0; j < RPL; j++) asm volatile("" : "+v"(acc[i][j]));
      }
      if (G & 1) __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <int T, class Fetch>
__device__ __forceinline__ void q4_tile896f(Fetch fetch, const PrepLds<T>& P, int lane, float acc[4]) {
  q4_tiles896f<T, 1>([&](int, int cb, uint4& w, uint2& s) { fetch(cb, w, s); }, P, lane, (float(*)[4])acc);
}

// Tile held in registers (lm_head stream).
template <int T>
__device__ __forceinline__ void q4_tile896(const Q4Tile& t, const PrepLds<T>& P, int lane, float acc[4]) {
  q4_tile896f<T>([&](int cb, uint4& w, uint2& s) { w = t.w[cb]; s = t.s[cb]; }, P, lane, acc);
}

// Tile staged in LDS in the HBM block layout: 7 x 1 KiB weights at `w`, 7 x 128 B scales at `s`.
template <int T>
__device__ __forceinline__ void q4_tile896_lds(const uint8_t* w, const uint8_t* s, const PrepLds<T>& P, int lane, float acc[4]) {
  const int n = lane & 15;
  q4_tile896f<T>([&](int cb, uint4& wv, uint2& sv) {
    wv = *(const uint4*)(w + cb * 1024 + lane * 16);
    sv = *(const uint2*)(s + cb * 128 + n * 8);
  }, P, lane, acc);
}

// NT tiles staged in LDS one after the other, `stride` bytes apart, each as
// [7 x 1 KiB weights][7 x 128 B scales].
template <int T, int NT>
__device__ __forceinline__ void q4_tiles896_lds(const uint8_t* base, int stride, const PrepLds<T>& P, int lane, float (*acc)[4]) {
  const int n = lane & 15;
  q4_tiles896f<T, NT>([&](int i, int cb, uint4& wv, uint2& sv) {
    wv = *(const uint4*)(base + i * stride + cb * 1024 + lane * 16);
    sv = *(const uint2*)(base + i * stride + ILL_KST * 1024 + cb * 128 + n * 8);
  }, P, lane, acc);
}
