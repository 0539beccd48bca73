// The pass kernel: one persistent launch runs a whole decode step, prefill chunk or
// tree-verify pass over T rows (T = 1 or 16 at compile time; `nrows` <= T at run time).
//
// The reference encodes the same work as 24 x 5 + 2 dependent dispatches
// (Sources/Engine/Engine.swift:245-292, :605-609). Here 256 workgroups stay resident and
// each layer is two dependent stages:
//
//   ATT[h]   (14 WGs, one per query head h, KV group g = h / 7)
//            x_l -> RMSNorm -> rows of q_h, k_g, v_g (+ bias, RoPE) -> MFMA flash attention
//            over 64-position chunks -> O projection restricted to head h's 64 columns
//            (split K) -> adds its 896-row partial into the residual accumulator XA[l]
//   GUD[ub]  (76 WGs, 64 hidden units each)
//            x'_l = XA[l] -> RMSNorm -> gate/up rows -> SiLU * up -> down projection
//            restricted to the 64 units (split K) -> adds into XB[l] (= x_{l+1})
//   LMH      (all WGs) final RMSNorm -> tied lm_head tiles -> per-WG argmax partials
//   COMMIT   (WG 0) argmax (ties -> lowest id), token record, state advance, tree accept,
//            KV compaction, epoch advance
//
// Residual accumulators hold 64-bit fixed point with the number of contributions in the
// top byte: each contributor adds (1 << 56) + (rint(v * 2^24) + 2^48). Integer addition
// makes the sum independent of arrival order (deterministic, and the same for any T), and
// a consumer knows an element is complete when its count reaches the number of
// contributors. A separate BASE workgroup adds the incoming residual as one more
// contributor.
// Accumulators alternate between two banks by pass; the idle bank is zeroed during the
// lm_head phase.
//
// Every role issues its weight loads for the next layer as soon as it has finished the
// current one, so HBM streaming overlaps the dependency chain.
#pragma once
#include "ill_device.h"

#define ILL_NATT 14          // ATT workgroups (one per query head)
#define ILL_R_ATT0 0         // ATT WGs 0..13
#define ILL_R_BASE 14        // the residual-copy workgroup
#define ILL_R_GUD0 16        // GUD WGs 16..91
#define ILL_R_PREP0 92       // 16-row passes: PREP WGs 92..107 (one per row)
#define ILL_RED_Q 8          // 16-row passes: REDUCE WGs per row
#define ILL_NRED (ILL_RED_Q * ILL_MAXT)
#define ILL_R_RED0 108       // 16-row passes: REDUCE WGs 108..235 (row r / 8, column eighth r % 8)
#define ILL_R_ATT1 236       // 16-row passes: ATT WGs 236..249, rows 8-15 of head wg - 236
#define ILL_R_IDLE0 92       // 1-row passes: WGs 92..255 have no layer role; each stages
#define ILL_LMH_PRE 16       // ILL_LMH_PRE lm_head tiles (two per wave) in its LDS meanwhile

struct IllPassArgs {
  IllWeights W;
  const IllLayerW* L;
  IllState* st;
  IllCtl* ctl;
  int32_t* ptoks;          // [16] row tokens of the pass (commit writes [0] for the next step)
  int32_t* tree;           // [65] (written by the host or the learned drafter)
  const float2* rope;      // [maxctx + 16][32] (cos, sin)
  uint16_t* kc;            // K cache [layer][kvh][maxctx][64] f16 (q8 / f16 engines: swizzled, ill_common.h)
  uint16_t* vt;            // V cache transposed per 64 slots [layer][kvh][maxctx/64][64 dims][64] f16 (idem)
  uint64_t* acc;           // residual accumulators [bank 2][layer][A/B][16][896]
  uint64_t* lmp;           // [256][16][2] lm_head argmax partials (value, index)
  float* logits;           // [16][V]
  int32_t* out_dev;        // [maxsteps]
  int32_t* out_host;       // [maxsteps] pinned host memory
  uint64_t* trace;         // optional [256][ILL_TRACE_SLOTS] timestamps (nullptr = off)
  uint64_t* pub;           // 16-row passes: published row codings [2][ILL_MAXLAYERS + 1][16][ILL_PUB_W]
  uint4* part;             // 16-row passes: down-projection partials [2][76][16][ILL_PART_ROW] checked words
  const uint4* ngram;      // optional n-gram draft table [ILL_NG_SLOTS] (nullptr: none)
  const int32_t* prompt;   // [4 + ILL_OB_MAX]: count, -, -, -, the last <= 256 prompt tokens
  int32_t* spec_host;      // pinned host [2]: passes and accepted drafts of speculative commits
  const int32_t* stop_host;   // pinned host word: nonzero once the host asked queued passes to stop
  int maxctx;
  int maxsteps;
  IllLayerW L0;            // L[0] again: the pass's first weight stage reads these pointers from
                           // the kernel arguments (scalar loads), not with a round trip each
};

// Layer l's weight pointers read with scalar loads (the table is written by the host only,
// so the constant address space is exact). Passes of 4 and 16 rows use them: a vector load
// of a pointer is waited for with vmcnt, which also waits for every weight stage the wave
// issued before it (16-row verify 4 us faster). The 1-row kernel keeps the generic loads:
// there the pointers' SGPRs spill into VGPR lanes in the role loops (10 us slower).
__device__ __forceinline__ IllLayerW layer_ptrs(const IllLayerW* L, int l) {
  static_assert(sizeof(IllLayerW) % 8 == 0, "pointer fields");
  typedef const __attribute__((address_space(4))) uint64_t* CP;
  const CP p = (CP)(L + l);
  uint64_t v[sizeof(IllLayerW) / 8];
#pragma unroll
  for (int i = 0; i < (int)(sizeof(IllLayerW) / 8); i++) v[i] = p[i];
  IllLayerW r;
  __builtin_memcpy(&r, v, sizeof r);
  return r;
}

// Trace slots per workgroup: ILL_TRL per layer (0 role start, 1 input ready, 2-10 and
// 12-15 role-specific intermediate points, 11 done) and 12 for the lm_head / commit tail
// (tail + 8: the workgroup entered the kernel, + 9: header loaded, + 10: it leaves).
#define ILL_TRL 16
#define ILL_TR_TAIL (ILL_TRL * ILL_MAXLAYERS)
#define ILL_TRACE_SLOTS (ILL_TR_TAIL + 12)
__device__ __forceinline__ void trace_mark(const IllPassArgs& a, int slot) {
  if (a.trace && threadIdx.x == 0) a.trace[blockIdx.x * ILL_TRACE_SLOTS + slot] = wall_clock64();
}

#define ILL_ERR_SHAPE 990   // error code: a pass's rows do not fit the kernel instantiation

struct PassHdr {
  uint32_t epoch;
  int mode, nrows, pos, lmh0, lmhn, wlog, commit, done, bank, zrows;
  int step, maxsteps, eos0, eos1, passes, accepted;   // State as the pass found it
  int tspec, nodraft;
  int tok[16], depth[16], parent[16];
  int prow[16][16];        // prow[t][d]: pass row on row t's path at depth d
};

// threadIdx.x passed through an opaque move. Address arithmetic derived from it then stays
// inside the role that uses it: without this the compiler hoists every per-lane address
// out of the layer loop, where the values occupy registers for the whole kernel.
__device__ __forceinline__ int tid_opaque() {
  int v = threadIdx.x;
  asm volatile("" : "+v"(v));
  return v;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations but not for
// its outstanding global loads, stores, atomics or LDS DMA (which __syncthreads would).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The pass header: State, control block and row metadata. Called by every thread of the
// workgroup (it holds two barriers). Wave 0's lanes load one word each (lanes 0-15 the
// State, 16-31 the control block, 32-47 the row tokens, 48-63 the tree's depths and
// parents), so the whole header is one round trip to memory; threads 0-15 then fill one
// row each of the path table. (Thread 0 filling it alone took 8.7 us at the start of every
// pass: its header reads became scalar loads, which share the lgkmcnt counter with LDS
// stores, so the waits for its ~150 LDS stores also waited for loads in flight, and the
// reads went out in six dependent rounds.)
__device__ __forceinline__ void load_hdr(const IllPassArgs& a, PassHdr& H) {
  __shared__ int raw[80];
  const int t = threadIdx.x;
  if (t < 64) {
    int v0, v1 = 0;
    if (t < 16) v0 = gld((const int32_t*)a.st + t);
    else if (t < 32) v0 = gld((const int32_t*)a.ctl + (t - 16));
    else if (t < 48) v0 = gld(a.ptoks + (t - 32));
    else {
      v0 = gld(a.tree + ILL_TR_DEPTH + (t - 48));
      v1 = gld(a.tree + ILL_TR_PARENT + (t - 48));
    }
    raw[t] = v0;
    if (t >= 48) raw[t + 16] = v1;
  }
  lds_barrier();
  const IllState& st = *(const IllState*)&raw[0];
  const IllCtl& c = *(const IllCtl*)&raw[16];
  const int mode = c.mode, nrows = c.nrows;
  static_assert(sizeof(IllState) == 64 && sizeof(IllCtl) == 64, "one word per lane");
  if (t == 0) {
    H.done = st.done;
    H.step = st.step;
    H.maxsteps = st.maxsteps;
    H.eos0 = st.eos0;
    H.eos1 = st.eos1;
    H.passes = st.passes;
    H.accepted = st.accepted;
    H.tspec = st.tspec;
    H.nodraft = st.nodraft;
    H.pos = st.pos;
    const uint32_t ep = c.epoch;
    H.epoch = ep;
    H.bank = ep & 1;
    H.zrows = (ep & 1) ? c.bank_rows[0] : c.bank_rows[1];
    H.mode = mode;
    H.nrows = nrows;
    H.lmh0 = c.lmh_row0;
    H.lmhn = c.lmh_rows;
    H.wlog = c.write_logits;
    H.commit = c.commit;
  }
  if (t < 16) {
    // row r's depth and parent: the tree's entries in tree passes, a chain otherwise
    auto depth = [&](int r) { return mode == ILL_MODE_TREE ? (r < nrows ? raw[48 + r] : 0) : r; };
    auto parent = [&](int r) { return mode == ILL_MODE_TREE ? (r < nrows ? raw[64 + r] : 0) : (r > 0 ? r - 1 : 0); };
    H.tok[t] = t < nrows ? raw[32 + t] : 0;
    H.depth[t] = depth(t);
    H.parent[t] = parent(t);
    int row[16];
#pragma unroll
    for (int d = 0; d < 16; d++) row[d] = 0;
    int r = t;
    for (int d = depth(t); d >= 0; --d) {
      if (d < 16) row[d] = r;
      r = r > 0 ? parent(r) : 0;
    }
#pragma unroll
    for (int d = 0; d < 16; d++) H.prow[t][d] = row[d];
  }
  lds_barrier();
}

// ---- residual fixed point --------------------------------------------------------------
#define FX_COUNT (1ull << 56)
#define FX_BIAS (1ll << 48)
#define FX_SCALE 16777216.0f        // 2^24
#define FX_INV (1.0f / 16777216.0f)

// round(v * 2^24), clamped to |q| <= 2^47, as hi * 2^31 + lo with |lo| < 2^31: both parts
// are exact in float (lo is a sub-range of the 24 significant bits of the scaled value).
__device__ __forceinline__ int64_t fx_of(float v) {
  const float x = rintf(__builtin_amdgcn_fmed3f(v * FX_SCALE, -140737488355328.0f, 140737488355328.0f));
  const float hf = truncf(x * 4.656612873077393e-10f);   // 2^-31
  const float lf = fmaf(hf, -2147483648.0f, x);
  return (int64_t)(int)hf * 2147483648ll + (int64_t)(int)lf;
}
__device__ __forceinline__ uint64_t fx_word(int64_t q) { return FX_COUNT + (uint64_t)(q + FX_BIAS); }
// value of a completed accumulator word (count = n contributions)
__device__ __forceinline__ int64_t fx_value(uint64_t w) {
  const int64_t n = (int64_t)(w >> 56);
  return (int64_t)(w & ((1ull << 56) - 1)) - n * FX_BIAS;
}
__device__ __forceinline__ int fx_count(uint64_t w) { return (int)(w >> 56); }
__device__ __forceinline__ float fx_float(int64_t v) { return (float)v * FX_INV; }
__device__ __forceinline__ void fx_add(uint64_t* p, uint64_t w) {
  __hip_atomic_fetch_add((GAS unsigned long long*)p, (unsigned long long)w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Column c of an accumulator row sits ILL_ACC_STRIDE words after column c - 1, so that a
// stride above 1 spreads the contributors' atomics over more cache lines.
#ifndef ILL_ACC_STRIDE
#define ILL_ACC_STRIDE 1
#endif
#define ILL_ACC_ROW (ILL_H * ILL_ACC_STRIDE)
__device__ __forceinline__ size_t acc_col(int c) { return (size_t)c * ILL_ACC_STRIDE; }
__device__ __forceinline__ uint64_t* acc_ptr(const IllPassArgs& a, int bank, int l, int kind, int t) {
  return a.acc + ((((size_t)bank * a.W.layers + l) * ILL_NKIND + kind) * 16 + t) * ILL_ACC_ROW;
}
// Copies in use: 16-row passes read every word 16 times over, so they keep one of each.
// Kinds per layer: XA copies 0 .. xa_copies - 1, XB copies from ILL_XA_COPIES on.
template <int T>
__host__ __device__ constexpr int xa_copies() { return T == 1 ? ILL_XA_COPIES : 1; }
// 16-row passes read their RMSNorm codings from PREP publications; passes of up to 4 rows
// code the accumulators themselves, as 1-row passes do.
template <int T>
__host__ __device__ constexpr bool ill_pub() { return T > 4; }
template <int T>
__host__ __device__ constexpr int xb_copies() { return T == 1 ? ILL_XB_COPIES : 1; }
#define ILL_KIND_XB ILL_XA_COPIES
// contributions expected in XA copy c (heads, plus the base in copy 0) and XB copy c
template <int T>
__device__ __forceinline__ int xa_expect(int c) { return ILL_NATT / xa_copies<T>() + (c == 0 ? 1 : 0); }
template <int T>
__device__ __forceinline__ int xb_expect(int c) { return ILL_NGU / xb_copies<T>() + (c == 0 ? 1 : 0); }

// ---- activation sources for prep896 --------------------------------------------------
// A residual accumulator: the sum of its copies (16 rows apart), complete when every copy
// has its contributions. XB = false: the post-attention residual XA[l] (kinds 0 ..), true:
// the post-MLP residual XB[l] (kinds ILL_KIND_XB ..).
// How a consumer polls an accumulator input (prep896): 0 the wave's light word (one column
// of each row) until it is complete, then the whole input; 1 the whole input every time;
// 2 the light word until it lacks at most ILL_SLACK_XA / ILL_SLACK_XB contributions, then
// the whole input (until complete).
// The slack is per accumulator (XA: 15 contributions at 16 rows, 8 / 7 per copy at one row;
// XB: 77, or 39 / 38): the full read is issued while the last contributions land, so it
// returns about when they are complete (one row, config 2: 333 -> 327.6 us per step with
// slack 4 / 8 against the plain two-stage poll; the full input every time: 339 us). With the
// watcher wave below, A/B in both orders on one box: 4 / 8 314.4-314.7 us, 2 / 4 314.8-314.9,
// 6 / 12 316.5-316.8 (the same tokens).
#ifndef ILL_POLL
#define ILL_POLL 2
#endif
// Inputs of prep896<1> from an accumulator: 1 = wave 0 alone polls the light words
// (ILL_POLL_D polls in flight, ILL_WATCH_SLEEP x 64 cycles between rounds) while the other
// waves wait at an LDS barrier, then every wave reads its columns as before. A step
// (config 2, graph-replayed, A/B in both orders on one box): every wave polling 318.0-318.5
// us, one watcher 314.0-314.5 us. Fewer polls of words that the atomics are updating is what
// pays (the workgroups' spread in the trace did not shrink): two or three watcher polls in
// flight 316.9-317.1 / 320.2-320.4 us, sleeps of 8 or 16 314.7-314.9 / 315.6-315.9 us, a
// watcher waiting for the complete word (no slack) 319.5 us.
#ifndef ILL_WATCH
#define ILL_WATCH 1
#endif
#ifndef ILL_POLL_D
#define ILL_POLL_D 1
#endif
#ifndef ILL_WATCH_SLEEP
#define ILL_WATCH_SLEEP 4
#endif
// 16-row REDUCE: 1 = one watcher wave polls a word of producers 0-12, the rest wait at a
// barrier, then every thread reads its words (0: every thread polls its own word first).
// 16-row verify at prefix 512, A/B in three rounds: 818.6-820.2 -> 816.6-817.1 us (median
// of 25 passes each), the same logits.
#ifndef ILL_WATCH_RED
#define ILL_WATCH_RED 1
#endif
#ifndef ILL_SLACK_XA
#define ILL_SLACK_XA 4
#endif
#ifndef ILL_SLACK_XB
#define ILL_SLACK_XB 8
#endif
template <int T, bool XB>
struct SrcRes {
  static constexpr int kSlack = XB ? ILL_SLACK_XB : ILL_SLACK_XA;
  static constexpr bool kPipe = true;
  static constexpr int NC = XB ? xb_copies<T>() : xa_copies<T>();
  struct Light {   // the light words of rows t < T, copies k < NC, in flight
    uint64_t w[T][NC];
  };
  const uint64_t* base;   // copy 0, row 0
  __device__ __forceinline__ void light_issue(Light& L, int nrows, int c) const {
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int k = 0; k < NC; k++)
        L.w[t][k] = t < nrows ? aload64(base + ((size_t)k * 16 + t) * ILL_ACC_ROW + acc_col(c)) : 0;
  }
  __device__ __forceinline__ bool light_check(const Light& L, int nrows, int slack) const {
    bool ok = true;
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
      for (int k = 0; k < NC; k++)
        if (t < nrows) ok &= fx_count(L.w[t][k]) + slack >= (XB ? xb_expect<T>(k) : xa_expect<T>(k));
    return ok;
  }
  // every copy of column c of row t lacks at most `slack` contributions
  __device__ __forceinline__ bool near1(int t, int c, int slack) const {
    constexpr int NC = XB ? xb_copies<T>() : xa_copies<T>();
    bool ok = true;
#pragma unroll
    for (int k = 0; k < NC; k++) {
      const uint64_t w = aload64(base + ((size_t)k * 16 + t) * ILL_ACC_ROW + acc_col(c));
      ok &= fx_count(w) + slack >= (XB ? xb_expect<T>(k) : xa_expect<T>(k));
    }
    return ok;
  }
  __device__ __forceinline__ bool load1(int t, int c, float& v) const {
    constexpr int NC = XB ? xb_copies<T>() : xa_copies<T>();
    bool ok = true;
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < NC; k++) {
      const uint64_t w = aload64(base + ((size_t)k * 16 + t) * ILL_ACC_ROW + acc_col(c));
      ok &= fx_count(w) == (XB ? xb_expect<T>(k) : xa_expect<T>(k));
      sum += fx_value(w);
    }
    v = fx_float(sum);
    return ok;
  }
};
template <int T>
using SrcXB = SrcRes<T, true>;
template <int T>
using SrcXA = SrcRes<T, false>;

// Embedding rows (layer-0 input), dequantized from the tiled q4 table: w = s*q + m
// (Shaders.swift:118-126 semantics).
__device__ __forceinline__ void embed16(const IllWeights& W, int tok, int c0, float* v) {
  const int rt = tok >> 4, n = tok & 15;
  const int cb = c0 >> 7, gi = (c0 >> 6) & 1, kg = (c0 >> 4) & 3;
  const uint8_t* blk = W.wemb + ((size_t)rt * ILL_KST + cb) * 1024 + (kg * 16 + n) * 16 + gi * 8;
  const uint2 b = gld((const uint2*)blk);
  const uint32_t sm = gld(W.semb + ((size_t)rt * ILL_KST + cb) * 32 + n * 2 + gi);
  const float s = h2f(sm & 0xffff), m = h2f(sm >> 16);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t word = i < 8 ? b.x : b.y;
    const uint32_t q = (word >> (4 * (i & 7))) & 0xF;
    v[i] = s * (float)q + m;
  }
}

__device__ __forceinline__ float embed1(const IllWeights& W, int tok, int c) {
  float v[16];
  embed16(W, tok, c & ~15, v);
  return v[c & 15];
}

struct SrcEmbed {
  static constexpr int kSlack = 0;
  static constexpr bool kPipe = false;
  IllWeights W;
  const int* toks;   // LDS copy of the row tokens
  __device__ __forceinline__ bool load1(int t, int c, float& v) const {
    v = embed1(W, toks[t], c);
    return true;
  }
  __device__ __forceinline__ bool near1(int, int, int) const { return true; }
};

__device__ __forceinline__ int q4perm_inv(int c) { return (c & 8) | ((c & 1) << 2) | ((c >> 1) & 3); }

// One row (64 values, one per lane) -> 16-bit coding as a K = 64 MFMA operand:
// lane (kg, m = row) of the operand holds units 16 kg + q4perm(p); operand k-group gi of
// row t is at [gi * T + t]. Lane c of a 16-lane row codes unit c, byte p = q4perm_inv(c)
// of its row's 16 bytes: the lanes c, c + 2, c + 4, c + 6 ((c & 6) == 0) fill bytes 0-3
// of dword ((c & 8) >> 2) | (c & 1), so two DPP row shifts gather each dword into one lane,
// which stores it.
#define ILL_DPP_SHL2 0x102   // row_shl:2 (lane l reads lane l + 2 of its row)
#define ILL_DPP_SHL4 0x104   // row_shl:4
template <int T>
__device__ __forceinline__ void quant_store(int qv, int t, uint4* ahi, uint4* alo, int lane) {
  const int hi = (qv + 128) >> 8, lo = qv - (hi << 8);
  uint32_t h = (uint32_t)hi & 0xff, l = (uint32_t)lo & 0xff;
  h |= (uint32_t)dpp_i<ILL_DPP_SHL2>((int)h) << 8;
  l |= (uint32_t)dpp_i<ILL_DPP_SHL2>((int)l) << 8;
  h |= (uint32_t)dpp_i<ILL_DPP_SHL4>((int)h) << 16;
  l |= (uint32_t)dpp_i<ILL_DPP_SHL4>((int)l) << 16;
  if ((lane & 6) == 0) {
    const int gi = lane >> 4, dw = ((lane & 8) >> 2) | (lane & 1);
    ((uint32_t*)&ahi[gi * T + t])[dw] = h;
    ((uint32_t*)&alo[gi * T + t])[dw] = l;
  }
}
// The codes of a group: v = rint(x * 32639 / max|x|) (0 for an all-zero group).
__device__ __forceinline__ int quant_code(float x, float mx) {
  return (int)rintf(x * (mx > 0.f ? ILL_QMAX * __builtin_amdgcn_rcpf(mx) : 0.f));
}
template <int T>
__device__ __forceinline__ void quant_row64(float h, int t, uint4* ahi, uint4* alo, float2* dsc, int lane) {
  const float mx = gmaxabs<64>(h);
  const int qv = quant_code(h, mx);
  const int sq = gsumi<64>(qv);
  quant_store<T>(qv, t, ahi, alo, lane);
  const float d = mx * (1.0f / ILL_QMAX);
  if (lane == 0) dsc[t] = make_float2(d, d * (float)sq);
}

// RMSNorm + 16-bit fixed-point coding of rows 0..nrows-1 of a K = 896 input into MFMA
// operands, spread over the whole workgroup: wave w owns column groups w and w + 8 (< 14)
// of every row, one column per lane. Every wave polls its own columns until they are
// complete, so the input is taken one memory round trip after its last contribution
// lands. Rows >= nrows are coded as zeros. The norm scale of a row is one positive factor
// of the whole row, so it is left out of the coding and applied to the products: per row,
// u = x * gamma is coded per group as v = rint(u * 32639 / max|u|) with step
// d = max|u| / 32639, all before the workgroup's one barrier, and the row's scale
// rsqrt(ss / 896 + eps) (ss = the waves' sums of squares of x, in order) is returned in
// rs[j] for rows 4 kg + j of this lane: callers multiply each product of the row by it.
// The sequence for a row does not depend on T.
template <int T, class Src>
__device__ __forceinline__ bool prep896(const Src& src, const float* gamma, int nrows, PrepLds<T>& P,
                                        IllCtl* ctl, int code, const IllPassArgs& a, float rs[4], int trs = -1) {
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int G1 = w + ILL_WAVES;
  const bool two = G1 < 14;   // wave-uniform
  const int c0 = 64 * w + lane, c1 = 64 * (two ? G1 : w) + lane;
  const float g0 = gld(gamma + c0), g1 = gld(gamma + c1);
  float v0[T], v1[T];
  const int cl = vgpr_uniform(64 * w);   // light poll: the wave's first column of each row
  auto full = [&]() {
    bool ok = true;
#pragma unroll
    for (int t = 0; t < T; t++) {
      v0[t] = 0.f;
      v1[t] = 0.f;
      if (t < nrows) {
        ok &= src.load1(t, c0, v0[t]);
        if (two) ok &= src.load1(t, c1, v1[t]);
      }
    }
    return ok;
  };
  bool alive;
  if constexpr (T == 1 && ILL_WATCH && Src::kPipe) {
    // wave 0 watches the light words; its verdict, written just before the barrier, is read
    // after it, so no earlier value of the word is ever taken for it
    using LW = typename Src::Light;
    if (w == 0) {
      const bool lit = wave_light_p<ILL_POLL_D, ILL_WATCH_SLEEP, LW>([&](LW& L) { src.light_issue(L, nrows, cl); },
                                                    [&](const LW& L) { return src.light_check(L, nrows, Src::kSlack); },
                                                    ctl, code);
      if (lane == 0) P.lit = lit;
    }
    lds_barrier();
    alive = P.lit && wave_wait(full, ctl, code);
  } else {
    alive = wave_wait2([&]() {
      bool ok = true;
      float x;
#pragma unroll
      for (int t = 0; t < T; t++)
        if (t < nrows) {
          if constexpr (ILL_POLL == 0) ok &= src.load1(t, cl, x);
          else if constexpr (ILL_POLL == 2) ok &= src.near1(t, cl, Src::kSlack);
        }
      return ok;
    }, full, ctl, code);
  }
  if (trs >= 0) trace_mark(a, trs);
  // stage by stage over blocks of up to 4 rows, so the rows' reduction chains interleave
  constexpr int RB = T < 4 ? T : 4;
#pragma unroll
  for (int t0 = 0; t0 < T; t0 += RB) {
    float u0[RB], u1[RB], m0[RB], m1[RB], ss[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) {
      const int t = t0 + r;
      ss[r] = gsum<64>(v0[t] * v0[t] + v1[t] * v1[t]);
      u0[r] = v0[t] * g0;
      u1[r] = v1[t] * g1;
      m0[r] = gmaxabs<64>(u0[r]);
      m1[r] = gmaxabs<64>(u1[r]);
    }
    int q0[RB], q1[RB], s0[RB], s1[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) {
      q0[r] = quant_code(u0[r], m0[r]);
      q1[r] = quant_code(u1[r], m1[r]);
      s0[r] = gsumi<64>(q0[r]);
      s1[r] = gsumi<64>(q1[r]);
    }
#pragma unroll
    for (int r = 0; r < RB; r++) {
      const int t = t0 + r;
      quant_store<T>(q0[r], t, P.ahi + w * 4 * T, P.alo + w * 4 * T, lane);
      if (two) quant_store<T>(q1[r], t, P.ahi + G1 * 4 * T, P.alo + G1 * 4 * T, lane);
      if (lane == 0) {
        P.red[w][t] = ss[r];
        const float d0 = m0[r] * (1.0f / ILL_QMAX);
        P.sc[w * T + t] = make_float2(d0, d0 * (float)s0[r]);
        if (two) {
          const float d1 = m1[r] * (1.0f / ILL_QMAX);
          P.sc[G1 * T + t] = make_float2(d1, d1 * (float)s1[r]);
        }
      }
    }
  }
  if (lane == 0) P.ok[w] = alive;
  if (trs >= 0 && (trs + 1) % ILL_TRL != 0) trace_mark(a, trs + 1);
  lds_barrier();
  const int4 ok0 = *(const int4*)&P.ok[0], ok1 = *(const int4*)&P.ok[4];
  // the row scales of this lane's rows 4 kg + j (at T = 1 every lane's row 0)
  const int kg = lane >> 4;
  constexpr int RPL = T >= 4 ? 4 : T;
#pragma unroll
  for (int j = 0; j < 4; j++) rs[j] = 1.f;
#pragma unroll
  for (int j = 0; j < RPL; j++) {
    const int t = arow<T>(4 * kg + j);
    float sst = 0.f;
#pragma unroll
    for (int ww = 0; ww < ILL_WAVES; ww++) sst += P.red[ww][t];
    rs[j] = __builtin_amdgcn_rsqf(sst * (1.0f / (float)ILL_H) + ILL_EPS);
  }
  return (ok0.x & ok0.y & ok0.z & ok0.w & ok1.x & ok1.y & ok1.z & ok1.w) != 0;
}

// ---- published codings (16-row passes) ----------------------------------------------------
// Every consumer of an accumulator needs all of its rows coded. In a 16-row pass that is
// 16 x 896 fixed-point words (114 KB) per consumer workgroup, read by 14 ATT, 76 GUD and
// 256 lm_head workgroups, each then running the same RMSNorm coding over 16 rows. Instead,
// one PREP workgroup per row runs prep896 on its row once (the arithmetic of a 1-row pass,
// so codes, group scales and row scale are bit-identical to it) and publishes the result,
// ILL_PUB_PAY payload dwords k:
//   [0, 224)    A-operand high bytes, 56 uint4 (column group g, k-group gi at 4 g + gi)
//   [224, 448)  low bytes
//   [448, 476)  group scales, 14 float2 (d, d * sum of the codes)
//   476         the row scale rsqrt(ss / 896 + eps)
// in ILL_PUB_Q 128-bit words: word m = 32 j + r (j < 5, r < 32) holds payload dwords
// k = 32 (3 j + i) + r, i < 3 (zero past 476), and a check dword tag ^ pub_mix(the three),
// tag = epoch * 32 + slot + 1. A word left from another epoch fails the check (its tag
// differs); one read torn between its halves fails it unless the mix collides (about 1 in
// 2^32). Words are written and read whole at device scope (sc1), and a consumer polls until
// every word it reads passes, so no ordering between the words is assumed.
// Consumer half-wave r reads row r: its lane's 5 words are the payload dwords lane + 32 j'
// (j' < 15) in order, which place into PrepLds<16> by shifts alone (16 rows: 40 KB).
// Buffers: kind 0 holds the GUD inputs (slot l: XA[l] under ln2), kind 1 the ATT inputs
// (slot l: x_l under ln1) and the final norm (slot = layers).
#define ILL_PUB_PAY 477
#define ILL_PUB_Q 160                       // 128-bit words per row
#define ILL_PUB_W (ILL_PUB_Q * 2)           // in 64-bit units
#define ILL_PUB_LIGHT 156                   // the word holding the row scale (k = 476)
#define ILL_PUB_WORDS (2 * (ILL_MAXLAYERS + 1) * ILL_MAXT * ILL_PUB_W)
#define ILL_BUF_SC1 16   // buffer access cache policy: device scope (sc1)
#define ILL_BUF_SYS 17   // system scope (sc0 sc1): memory the host writes
typedef uint32_t ill_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t tagof_pub(uint32_t epoch, int slot) { return epoch * 32u + (uint32_t)slot + 1u; }
__device__ __forceinline__ uint64_t* pub_ptr(const IllPassArgs& a, int kind, int slot, int t) {
  return a.pub + (((size_t)kind * (ILL_MAXLAYERS + 1) + slot) * ILL_MAXT + t) * ILL_PUB_W;
}
__device__ __forceinline__ uint32_t pub_mix(uint32_t x, uint32_t y, uint32_t z) {
  uint32_t h = x * 0x9E3779B1u;
  h = (h ^ (h >> 15)) + y * 0x85EBCA77u;
  h = (h ^ (h >> 13)) + z * 0xC2B2AE3Du;
  return h ^ (h >> 16);
}
__device__ __forceinline__ bool pub_ok(const ill_v4u& q, uint32_t tag) { return q[3] == (tag ^ pub_mix(q[0], q[1], q[2])); }
// byte-addressed buffer resource over n bytes from p (raw, untyped dword access)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pub_rsrc(const void* p, int n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, n, 0x00020000);
}

// Publish a 1-row coding (PrepLds<1> as prep896<1> left it, rs = its row scale): thread m
// writes word m.
__device__ __forceinline__ void pub_write(const PrepLds<1>& P, float rs, uint64_t* dst, uint32_t tag) {
  static_assert(offsetof(PrepLds<1>, ahi) == 0 && offsetof(PrepLds<1>, alo) == 896 && offsetof(PrepLds<1>, sc) == 1792,
                "payload dwords 0 .. 475 contiguous");
  const int m = tid_opaque();
  if (m < ILL_PUB_Q) {
    const uint32_t* pw = (const uint32_t*)P.ahi;
    uint32_t x[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const int k = 32 * (3 * (m >> 5) + i) + (m & 31);
      x[i] = k < 476 ? pw[k] : (k == 476 ? __float_as_uint(rs) : 0u);
    }
    const ill_v4u q = {x[0], x[1], x[2], tag ^ pub_mix(x[0], x[1], x[2])};
    __builtin_amdgcn_raw_buffer_store_b128(q, pub_rsrc(dst, ILL_PUB_Q * 16), m * 16, 0, ILL_BUF_SC1);
  }
}

// The consumer side: rows 0 .. nrows - 1 of a published coding (src = row 0) into P, as
// prep896<T> would have left it (rows >= nrows coded as zeros), and the row scales of this
// lane's rows 4 kg + j in rs[j]. Half-wave r of the workgroup reads row r: payload dwords
// lane + 32 j (j < 15) into v[j]; for j < 14 the dword's kind (high / low bytes) and place
// follow from j and the lane by shifts, so placing it costs no division.
template <int T>
__device__ __forceinline__ bool pub_read(const uint64_t* src, uint32_t tag, int nrows, PrepLds<T>& P, IllCtl* ctl,
                                         int code, const IllPassArgs& a, float rs[4], int trs = -1) {
  static_assert(T == ILL_MAXT && ILL_PUB_Q == 5 * 32 && T * 32 == ILL_WG_THREADS, "one half-wave per row");
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int t = tid >> 5, l32 = tid & 31;
  const bool live = t < nrows;
  const __amdgpu_buffer_rsrc_t rsrc = pub_rsrc(src, ILL_MAXT * ILL_PUB_Q * 16);
  const int rbase = t * (ILL_PUB_Q * 16) + l32 * 16;
  uint32_t v[15];
  // light poll: the word of the row scale, the same address for the half-wave. (Offsets
  // pass through opq, so every poll issues its loads afresh.) The first full read goes
  // through the L2 (no sc1): the consumers on one XCD then share one fetch of each line.
  // A line the L2 held from before the write fails the check (its words carry another
  // tag, or miss part of it), and every later read is at device scope.
  bool cached = true;
  const bool alive = wave_wait2([&]() {
    if (!live) return true;
    return pub_ok(__builtin_amdgcn_raw_buffer_load_b128(rsrc, opq(t * (ILL_PUB_Q * 16) + ILL_PUB_LIGHT * 16), 0, ILL_BUF_SC1), tag);
  }, [&]() {
    bool ok = true;
    ill_v4u q[5];
#pragma unroll
    for (int j = 0; j < 5; j++) {
      q[j] = (ill_v4u){0u, 0u, 0u, 0u};
      if (live) {
        if (cached) q[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, opq(rbase + j * 512), 0, 0);
        else q[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, opq(rbase + j * 512), 0, ILL_BUF_SC1);
      }
    }
    cached = false;
#pragma unroll
    for (int j = 0; j < 5; j++) {
      if (live) ok &= pub_ok(q[j], tag);
      v[3 * j] = q[j][0];
      v[3 * j + 1] = q[j][1];
      v[3 * j + 2] = q[j][2];
    }
    return ok;
  }, ctl, code);
  if (trs >= 0) trace_mark(a, trs);
#pragma unroll
  for (int j = 0; j < 14; j++) {   // codes: dword k = 32 j + l32 is dword k % 4 of uint4 k / 4 (group, k-group)
    const int k = (j % 7) * 32 + l32;
    uint32_t* dst = (uint32_t*)(j < 7 ? P.ahi : P.alo);
    dst[((k >> 2) * T + t) * 4 + (k & 3)] = v[j];
  }
  if (l32 < 28) ((uint32_t*)P.sc)[((l32 >> 1) * T + t) * 2 + (l32 & 1)] = v[14];
  else if (l32 == 28) P.red[0][t] = live ? __uint_as_float(v[14]) : 1.f;
  if (lane == 0) P.ok[w] = alive;
  lds_barrier();
  const int4 ok0 = *(const int4*)&P.ok[0], ok1 = *(const int4*)&P.ok[4];
  const int kg = lane >> 4;
#pragma unroll
  for (int j = 0; j < 4; j++) rs[j] = P.red[0][arow<T>(4 * kg + j)];
  return (ok0.x & ok0.y & ok0.z & ok0.w & ok1.x & ok1.y & ok1.z & ok1.w) != 0;
}

// ---- weight staging in LDS ----------------------------------------------------------------
// Each role copies the next layer's weights HBM -> LDS (global_load_lds) as soon as it has
// finished the current layer, per wave, into a dynamic-LDS stage of ILL_STAGE_BYTES:
//   ATT  QKV: row tile lt (0-11) at lt * 8064: [7 KiB codes][7 x 128 B scales], staged by
//             the wave that computes it
//        O:   wave w at w * 4032: [7 row tiles x 512 B][7 x 64 B scales] (loaded after QKV)
//   GUD  GU:  wave w at w * 8064: [7 KiB][896 B]
//        down: wave w at 64512 + w * 4032: [7 x 512 B][7 x 64 B]
#define ILL_STAGE_BYTES 96768
#define ILL_ST_TILE 8064
// At T = 1 the static LDS is small, so the ATT role keeps its O weights in a region of
// their own after the QKV block and stages both at the end of the previous layer.
__host__ __device__ constexpr int ill_stage_bytes(int T) { return T == 1 ? ILL_STAGE_BYTES + 8 * 4032 : ILL_STAGE_BYTES; }
__host__ __device__ constexpr int ill_st_o(int T) { return T == 1 ? ILL_STAGE_BYTES : 0; }
#define ILL_ST_SPLIT 4032
#define ILL_ST_GU 8064
#define ILL_ST_DOWN0 64512

// Split-K partial of a 896-row projection over one 64-column group: the wave's 7 row
// tiles (rows 112 w .. +112) of a [group][row tile] 512-byte block layout, staged in LDS.
__device__ __forceinline__ void split_stage(const uint8_t* wg, const uint32_t* sg, int w, int lane, uint8_t* dst) {
  wave_copy_to_lds(wg + (size_t)(7 * w) * 512, dst, 7 * 512, lane);
  wave_copy_to_lds((const uint8_t*)(sg + 7 * w * 16), dst + 7 * 512, 7 * 64, lane);
}

// ---------------------------------------------------------------------------------------
template <int T>
struct AttLds {
  union {
    PrepLds<T> prep;
    float P[ILL_WAVES][T][64];
    struct {
      float cm[ILL_WAVES][T], cl[ILL_WAVES][T];
      float co[ILL_WAVES][T][64];
    } c;
  } u;
  float q[T][64];
  uint16_t k[T][64];
  uint16_t v[T][64];
  float pm[2][T], pl[2][T];   // statistics of the partial chunks ns + i per row
  float po[2][T][64];
  uint4 ahi[4 * T], alo[4 * T];
  float2 dsc[T];
  float p1[T == 1 ? ILL_WAVES : 1][64];   // T = 1: the waves' P scratch, outside the union
};

// Per-wave scratch [T][64] for a chunk's probabilities. At T = 1 it lies outside the region
// the combine state reuses, so no barrier separates the last chunk from the state writes.
template <int T>
__device__ __forceinline__ float* att_pbuf(AttLds<T>& A, int w) { return T == 1 ? &A.p1[w][0] : &A.u.P[w][0][0]; }

template <int T>
struct GudLds {
  PrepLds<T> prep;
  float gu[8][T][16];
  uint4 ahi[4 * T], alo[4 * T];
  float2 dsc[T];
  // T = 1: each wave's own coding of the SiLU row (wave w at [4 w], [w])
  uint4 wahi[T == 1 ? 4 * ILL_WAVES : 1], walo[T == 1 ? 4 * ILL_WAVES : 1];
  float2 wdsc[T == 1 ? ILL_WAVES : 1];
};

template <int T>
struct LmhLds {
  PrepLds<T> prep;
  float bv[ILL_WAVES][16];
  int bi[ILL_WAVES][16];
};

// Speculative drafting after a commit (k_commit_spec, Shaders.swift:367-412): recent output
// tokens, the n-gram history, and the workgroup's reduction slots.
#define ILL_OB_MAX 256
#define ILL_NG_SLOTS (1 << 20)
#define ILL_NG_MAXN 6
struct DraftLds {
  int ob[ILL_OB_MAX + ILL_MAXT];   // recent output tokens, then this commit's drafts
  int hist[ILL_NG_MAXN + ILL_MAXT];
  uint32_t best[ILL_WAVES];
  int ng[ILL_NG_MAXN][16];          // n-gram probes: 0 occupied by another key, 1 empty, 2 + next: hit
  int L, len, d, nd;
};

struct CommitLds {
  uint64_t key[16][ILL_WG / 64];   // [row - first row][wave holding the row's partials]
  int g[16];
  int path[16];
  int npath, pos0;
};

template <int T>
union PassLds {
  AttLds<T> att;
  GudLds<T> gud;
  LmhLds<T> lmh;
  PrepLds<1> prep1;
  CommitLds cm;
};

// ATT workgroup weights: six 32-row QKV blocks bw (q_h halves, k_g halves, v_g halves;
// att_block gives the block of the fused matrix) and every wave 7 row tiles of O's head-h
// columns. Row tile lt = 2 bw + hf is half hf of block bw (dims d, or d + 32, of the head,
// d = 16 (block & 1) + n). Wave w computes qkv_nt(w) tiles from qkv_lt0(w):
// waves 0-3 both halves of blocks 0-3 (q and k: a RoPE pair stays in one lane), waves 4-7
// one half of a v block each, so each SIMD (waves w, w + 4) runs 3 tiles. (At T > 1 the
// tiles are bound by their per-group epilogue arithmetic, which this spreads evenly.)
__device__ __forceinline__ int att_block(int h, int bw) {
  const int g = h / 7;
  return bw < 2 ? 2 * h + bw : (bw < 4 ? 28 + 2 * g + (bw - 2) : 32 + 2 * g + (bw - 4));
}
template <int T>
__device__ __forceinline__ int qkv_nt(int w) { return w < 4 ? 2 : 1; }
template <int T>
__device__ __forceinline__ int qkv_lt0(int w) { return w >= 4 ? w + 4 : 2 * w; }

template <int T>
__device__ __forceinline__ void att_stage_qkv(const IllLayerW& L, int h, int w, int lane, uint8_t* stage) {
  const int nt = qkv_nt<T>(w), lt0 = qkv_lt0<T>(w);
  for (int i = 0; i < nt; i++) {
    const int lt = lt0 + i;
    const int r = 2 * att_block(h, lt >> 1) + (lt & 1);   // row tile of the fused QKV matrix
    uint8_t* d = stage + lt * ILL_ST_TILE;
    wave_copy_to_lds(L.wqkv + (size_t)r * ILL_KST * 1024, d, ILL_KST * 1024, lane);
    wave_copy_to_lds((const uint8_t*)(L.sqkv + r * ILL_KST * 32), d + ILL_KST * 1024, ILL_KST * 128, lane);
  }
}

// Attention work is dealt out by slot: slot j holds the shared chunks c = j (mod 8) and the
// partial pairs numbered j - ns (mod 8). Slot j runs on wave (j + 4) % 8, so the shared
// chunks go first to the waves with one QKV tile. (The mapping is its own inverse.)
template <int T>
__device__ __forceinline__ int att_slot(int w) { return (w + 4) & 7; }

template <int T>
__device__ __forceinline__ void att_stage_o(const IllLayerW& L, int h, int w, int lane, uint8_t* stage) {
  split_stage(L.wo + (size_t)h * ILL_NOT * 512, L.so + h * ILL_NOT * 16, w, lane, stage + ill_st_o(T) + w * ILL_ST_SPLIT);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ v8h u4_to_v8h(uint4 u) {
  v8h r;
  const uint32_t x[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    r[2 * i] = __builtin_bit_cast(_Float16, (unsigned short)(x[i] & 0xffff));
    r[2 * i + 1] = __builtin_bit_cast(_Float16, (unsigned short)(x[i] >> 16));
  }
  return r;
}
// Bitwise select (m = all ones or zero): keeps the compiler from turning a select of a
// loaded value into a branch around the load.
__device__ __forceinline__ uint32_t msel(uint32_t m, uint32_t a, uint32_t b) { return (a & m) | (b & ~m); }
__device__ __forceinline__ uint4 msel4(uint32_t m, uint4 a, uint4 b) {
  return make_uint4(msel(m, a.x, b.x), msel(m, a.y, b.y), msel(m, a.z, b.z), msel(m, a.w, b.w));
}
__device__ __forceinline__ uint32_t mask_of(bool c) { return 0u - (uint32_t)c; }

// e^x for the softmax as 2^(x log2 e) on the hardware exp2 (exp(-inf) = 0).
__device__ __forceinline__ float att_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// Pass-row V along each row's path, [T][64 dims][16 depths] u16 (zero beyond the row's
// depth), built in the free part of the weight stage before attention.
#define ILL_ST_VPT 32256

// ---- attention ------------------------------------------------------------------------
// Positions are split into 64-position chunks by virtual position (the position a key has
// on the row's own path), so a row's arithmetic depends only on its path and not on how
// the path is split between the cache and the rows of the current pass:
//   chunks c < ns = pos / 64 lie below pos and are shared by every row; chunk c goes to
//     wave c % 8, which folds its chunks into a running (max, sum, output) in order of c;
//   chunks c >= ns ("partial") hold pass rows. Each (chunk, row) pair is evaluated on its
//     own by some wave; its statistics are folded into wave c % 8's running state at the
//     combine, after that wave's shared chunks, i.e. still in order of c.
// At T = 1 the chunk holding the new position is the only partial chunk.

// One cache chunk as MFMA operands for this lane (kg, n):
// k[b][hf]: key 64c + 16b + n, dims 32 hf + 8 kg .. +8; v[nb][ks]: dim 16 nb + n,
// positions 64c + 32 ks + 8 kg .. +8 (from the transposed V layout).
struct KVFrag {
  uint4 k[4][2];
  uint4 v[4][2];
};

// SWZ: the cache in the swizzled layout of the q8 / f16 engines (ill_common.h; the same
// fragments, read as 256-byte runs); the pass kernel's cache is in rows.
template <bool SWZ = false>
__device__ __forceinline__ void kv_fetch(const uint16_t* kbase, const uint16_t* vbase, int c, int lane, KVFrag& f) {
  const int kg = lane >> 4, n = lane & 15;
  if constexpr (SWZ) {
#pragma unroll
    for (int b = 0; b < 4; b++) {
      f.k[b][0] = gld((const uint4*)(kbase + kv_k_off(64 * c + 16 * b + n, 8 * kg, true)));
      f.k[b][1] = gld((const uint4*)(kbase + kv_k_off(64 * c + 16 * b + n, 32 + 8 * kg, true)));
    }
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
#pragma unroll
      for (int ks = 0; ks < 2; ks++)
        f.v[nb][ks] = gld((const uint4*)(vbase + kv_v_off(64 * c + 32 * ks + 8 * kg, 16 * nb + n, true)));
    }
    return;
  }
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const uint4* kr = (const uint4*)(kbase + (size_t)(64 * c + 16 * b + n) * 64);
    f.k[b][0] = gld(kr + kg);
    f.k[b][1] = gld(kr + 4 + kg);
  }
#pragma unroll
  for (int nb = 0; nb < 4; nb++) {
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
      f.v[nb][ks] = gld((const uint4*)(vbase + ((size_t)c * 64 + 16 * nb + n) * 64 + 32 * ks + 8 * kg));
  }
}

// Chunk-local attention over positions 64c .. 64c+63. With `part` (1-row passes: the chunk
// holding pos), the key and value at pos are the pass row's and keys above pos are
// masked; without it every key is a valid cache key. Results for rows 4 kg + j of this
// lane: mx = max score, ls = sum exp(s - mx), o[nb] = sum exp(s - mx) v (dims 16 nb + n).
// (16-row passes evaluate their partial chunks with part_eval16.)
template <int T>
__device__ __forceinline__ void chunk_eval(const PassHdr& H, AttLds<T>& A, const uint8_t* stage, const KVFrag& f, int c, bool part,
                                           int t1, const v8h qa[2][2], float mx[4], float ls[4], float o[4][4]) {
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int pos = H.pos;
  const int Lt = part ? pos + H.depth[t1] + 1 : 0x7fffffff;
  const uint4 zz = make_uint4(0, 0, 0, 0);
  float* pb = att_pbuf<T>(A, w);
  // T = 1: the key at pos is the pass row's (from LDS; only block (pos - 64 c) / 16 holds
  // it); keys above pos are masked through their scores, so their cache contents are never
  // used
  uint4 kp0 = zz, kp1 = zz;
  if (T == 1 && part) {
    kp0 = *(const uint4*)&A.k[0][8 * kg];
    kp1 = *(const uint4*)&A.k[0][32 + 8 * kg];
  }
  float sc[4][4];
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const int vp = 64 * c + 16 * b + n;
    uint4 k0 = f.k[b][0], k1 = f.k[b][1];
    if (T == 1 && part) {
      if (b == ((pos - 64 * c) >> 4)) {   // wave-uniform
        const uint32_t mp = mask_of(vp == pos);
        k0 = msel4(mp, kp0, k0);
        k1 = msel4(mp, kp1, k1);
      }
    }
    v4f s = {0.f, 0.f, 0.f, 0.f};
    // T = 1: a key block wholly above pos is all masked; its MFMAs are skipped (wave-uniform)
    if (!(T == 1 && part && 16 * b > pos - 64 * c)) {
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][0], u4_to_v8h(k0), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][1], u4_to_v8h(k0), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][0], u4_to_v8h(k1), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][1], u4_to_v8h(k1), s, 0, 0, 0);
    }
    const bool valid = vp < Lt;
#pragma unroll
    for (int j = 0; j < 4; j++) sc[b][j] = valid ? s[j] : -INFINITY;
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float m = fmaxf(fmaxf(sc[0][j], sc[1][j]), fmaxf(sc[2][j], sc[3][j]));
    mx[j] = gmax<16>(m);
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    float sum = 0.f;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      sc[b][j] = att_exp(sc[b][j] - mx[j]);
      sum += sc[b][j];
    }
    ls[j] = gsum<16>(sum);
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int t = 4 * kg + j;
    if (t < T) {
#pragma unroll
      for (int b = 0; b < 4; b++) pb[t * 64 + 16 * b + n] = sc[b][j];
    }
  }
  wave_lds_sync();
  v8h ph[2], pl[2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float p = pb[arow<T>(n) * 64 + 32 * ks + 8 * kg + i];
      const _Float16 hi = (_Float16)p;
      ph[ks][i] = hi;
      pl[ks][i] = (_Float16)(p - (float)hi);
    }
  }
  wave_lds_sync();
  // T = 1: V at positions below pos from the cache, at pos the pass row's; positions above
  // pos keep their (finite: the cache stores saturated f16) cache values, which meet
  // probabilities of exactly 0. The one 32-bit word holding pos (wave-uniform ks, word and
  // half, lanes kg = (dp / 8) % 4) takes the pass row.
  const int dp = pos - 64 * c;
  uint32_t lv1[4] = {0u, 0u, 0u, 0u};   // T = 1: the pass row's V, read by every lane
  if (T == 1 && part) {
#pragma unroll
    for (int nb = 0; nb < 4; nb++) lv1[nb] = A.v[0][16 * nb + n];
  }
#pragma unroll
  for (int nb = 0; nb < 4; nb++) {
    const int dim = 16 * nb + n;
    v8h vv[2];
    const uint32_t hm = mask_of(kg == ((dp >> 3) & 3)) & (0xffffu << (16 * (dp & 1)));   // bits of pos
    const uint32_t lvs = lv1[nb] << (16 * (dp & 1));
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      uint4 u = f.v[nb][ks];
      if (T == 1 && part) {
        uint32_t x[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int wi = 0; wi < 4; wi++)
          if (ks == (dp >> 5) && wi == ((dp >> 1) & 3)) x[wi] = msel(hm, lvs, x[wi]);
        u = make_uint4(x[0], x[1], x[2], x[3]);
      }
      vv[ks] = u4_to_v8h(u);
    }
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[0], vv[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[0], vv[0], acc, 0, 0, 0);
    // T = 1: positions 32 .. 63 of the chunk all above pos hold p = 0 and finite v
    // (skipped; adding them would add zeros)
    if (!(T == 1 && part && dp < 32)) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[1], vv[1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[1], vv[1], acc, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) o[nb][j] = acc[j];
  }
}

// Folding chunk statistics (m2, l2, o2) into a running state (m, l, o) is the one rule
// used for every chunk of every row: mn = max(m, m2), sa = exp(m - mn), sb = exp(m2 - mn),
// o' = o sa + o2 sb, l' = l sa + l2 sb.
struct AttScale {
  float mn, sa, sb;
};
__device__ __forceinline__ AttScale att_scale(float m, float m2) {
  AttScale r;
  r.mn = fmaxf(m, m2);
  r.sa = att_exp(m - r.mn);
  r.sb = att_exp(m2 - r.mn);
  return r;
}
__device__ __forceinline__ float att_fold(float x, float x2, const AttScale& k) { return x * k.sa + x2 * k.sb; }

// The outputs of split_gemv's multi-row form before they are added: y[k][j] is row
// 4 kg + j, column 16 k + n of the wave's 112 (lane (kg, n)).
template <int T>
__device__ __forceinline__ void split_outputs(const uint8_t* so, const uint4* ahi, const uint4* alo, const float2* dsc,
                                              int lane, float (&y)[7][4]) {
  static_assert(T >= 4, "multi-row form");
  const int kg = lane >> 4, n = lane & 15;
  constexpr int RPL = 4;
  const uint4 xh = ahi[kg * T + arow<T>(n)];
  const uint4 xl = alo[kg * T + arow<T>(n)];
  const v4i ah = (v4i){(int)xh.x, (int)xh.y, (int)xh.z, (int)xh.w};
  const v4i al = (v4i){(int)xl.x, (int)xl.y, (int)xl.z, (int)xl.w};
  const v4i z = {0, 0, 0, 0};
  uint2 wv[7];
  uint32_t sm[7];
#pragma unroll
  for (int k = 0; k < 7; k++) {
    wv[k] = *(const uint2*)(so + k * 512 + lane * 8);
    sm[k] = *(const uint32_t*)(so + 7 * 512 + k * 64 + n * 4);
  }
  float2 dx[RPL];
#pragma unroll
  for (int j = 0; j < RPL; j++) dx[j] = dsc[arow<T>(4 * kg + j)];
#pragma unroll
  for (int k = 0; k < 7; k++) {
    const v4i bq = q4_unpack(wv[k].x, wv[k].y);
    const v4i dh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, bq, z, 0, 0, 0);
    const v4i dl = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, bq, z, 0, 0, 0);
    const float sw = h2f(sm[k] & 0xffff), mw = h2f(sm[k] >> 16);
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int Sv = (dh[j] << 8) + dl[j];
      float v = 0.f;
      v = fmaf(sw, dx[j].x * (float)Sv, v);
      v = fmaf(mw, dx[j].y, v);
      y[k][j] = v;
    }
  }
}

// Split-K partial of an 896-row projection over one 64-column input group (O: one head,
// down: 64 hidden units), from this wave's 7 staged row tiles (rows 112 w .. +112, LDS
// layout [7 x 512 B codes][7 x 64 B scales]). Each output y = s*d*S + m*X is added to
// row t < nrows of the accumulator (`accw` = row 0, element 112 w) as a fixed-point
// contribution. All operand reads and MFMAs come before the atomics.
// At T = 1 the lane rows alternate the high and low bytes of the one input row, so one
// MFMA per tile gives S in every lane: lane (kg, n) finishes only tiles kg and 4 + kg
// (< 7), two outputs and two atomics per lane where the 16-row form has seven of each.
// The arithmetic of each output is the same in both forms.
template <int T>
__device__ __forceinline__ void split_gemv(const uint8_t* so, const uint4* ahi, const uint4* alo, const float2* dsc,
                                           int lane, int nrows, uint64_t* accw, int rlo = 0) {
  const int kg = lane >> 4, n = lane & 15;
  constexpr int RPL = T >= 4 ? 4 : T;
  if constexpr (T == 1) {
    const uint4 x = ((lane & 1) ? alo : ahi)[kg];
    const v4i ax = (v4i){(int)x.x, (int)x.y, (int)x.z, (int)x.w};
    const v4i z = {0, 0, 0, 0};
    uint2 wv[7];
#pragma unroll
    for (int k = 0; k < 7; k++) wv[k] = *(const uint2*)(so + k * 512 + lane * 8);
    const int ka = kg, kb = 4 + min(kg, 2);
    const uint32_t sa = *(const uint32_t*)(so + 7 * 512 + ka * 64 + n * 4);
    const uint32_t sb = *(const uint32_t*)(so + 7 * 512 + kb * 64 + n * 4);
    const float2 dx = dsc[0];
    int S[7];
#pragma unroll
    for (int k = 0; k < 7; k++) {
      const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax, q4_unpack(wv[k].x, wv[k].y), z, 0, 0, 0);
      S[k] = (d[0] << 8) + d[1];
    }
    const int Sa = kg == 0 ? S[0] : kg == 1 ? S[1] : kg == 2 ? S[2] : S[3];
    const int Sb = kg == 0 ? S[4] : kg == 1 ? S[5] : S[6];
    auto out = [&](int Sv, uint32_t smv) {
      float v = 0.f;
      v = fmaf(h2f(smv & 0xffff), dx.x * (float)Sv, v);
      v = fmaf(h2f(smv >> 16), dx.y, v);
      return v;
    };
    const float ya = out(Sa, sa), yb = out(Sb, sb);
    fx_add(accw + acc_col(16 * ka + n), fx_word(fx_of(ya)));
    if (kg < 3) fx_add(accw + acc_col(16 * kb + n), fx_word(fx_of(yb)));
    return;
  }
  if constexpr (T > 1) {
    float y[7][4];
    split_outputs<T>(so, ahi, alo, dsc, lane, y);
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t >= rlo && t < nrows) {
#pragma unroll
        for (int k = 0; k < 7; k++) fx_add(accw + (size_t)t * ILL_ACC_ROW + acc_col(16 * k + n), fx_word(fx_of(y[k][j])));
      }
    }
  }
}

// ---- down-projection partials (16-row passes) -------------------------------------------
// GUD workgroup ub writes its partial y (rows t < nrows, 896 columns) as ILL_PART_ROW
// checked 128-bit words per row (the publications' format: three float32 payload dwords
// and tag ^ pub_mix): word (t, q, m), q < 8, m < 38, holds columns 112 q + 3 m + i, i < 3
// (the last two of word 37 are zero). Buffer half l & 1 serves layer l: a workgroup writes the
// partials of layer l + 2 only after XB[l] is complete, that is after every REDUCE read of
// layer l.
#define ILL_RED_COLS (ILL_H / ILL_RED_Q)          // columns per REDUCE workgroup (112)
#define ILL_PART_Q ((ILL_RED_COLS + 2) / 3)      // words per (row, REDUCE workgroup)
#define ILL_PART_ROW (ILL_RED_Q * ILL_PART_Q)
#define ILL_PART_WORDS (2 * ILL_NGU * ILL_MAXT * ILL_PART_ROW)
__device__ __forceinline__ void part_write(const IllPassArgs& a, uint32_t epoch, int l, int ub, const float* yt, int nrows) {
  const int tid = tid_opaque();
  const uint32_t tag = tagof_pub(epoch, l);
  const uint4* blk = a.part + ((size_t)((l & 1) * ILL_NGU + ub) * ILL_MAXT) * ILL_PART_ROW;
  const __amdgpu_buffer_rsrc_t r = pub_rsrc(blk, ILL_MAXT * ILL_PART_ROW * 16);
  for (int i = tid; i < nrows * ILL_PART_ROW; i += ILL_WG_THREADS) {
    const int t = i / ILL_PART_ROW, rem = i - t * ILL_PART_ROW, q = rem / ILL_PART_Q, m = rem - q * ILL_PART_Q;
    const float* src = yt + t * ILL_H + ILL_RED_COLS * q + 3 * m;
    const uint32_t x0 = __float_as_uint(src[0]);
    const uint32_t x1 = 3 * m + 1 < ILL_RED_COLS ? __float_as_uint(src[1]) : 0u;
    const uint32_t x2 = 3 * m + 2 < ILL_RED_COLS ? __float_as_uint(src[2]) : 0u;
    const ill_v4u wd = {x0, x1, x2, tag ^ pub_mix(x0, x1, x2)};
    __builtin_amdgcn_raw_buffer_store_b128(wd, r, i * 16, 0, ILL_BUF_SC1);
  }
}

// REDUCE (16-row passes, ILL_NRED workgroups; rows t >= nrows idle): workgroup r owns row
// t = r / 8, columns 112 q .. 112 q + 111 (q = r % 8), of the residual stream, in place of
// the BASE workgroup of shorter passes. First it adds the embedding into XA[0]; then, layer
// by layer, it sums the 76 partials of the down projection (their fx_of values, as the
// atomics of shorter passes would) and the completed XA[l], makes that total XB[l] in one
// contribution of count 77, and adds it into XA[l + 1] as the base of the next layer. The
// integers are the ones the per-partial atomics and the BASE copies would have produced.
// Threads (g, m), g < 13, m < 38, poll and sum word m of producers g, g + 13, ...; the 13
// sums of a word meet in LDS.
template <int T>
__device__ __forceinline__ bool role_red(const IllPassArgs& a, const PassHdr& H, int r, uint8_t* lds) {
  constexpr int NG = ILL_WG_THREADS / ILL_PART_Q, PER = (ILL_NGU + NG - 1) / NG;   // 13 groups of 6 producers
  const int t = r / ILL_RED_Q, q = r % ILL_RED_Q;
  if (t >= H.nrows) return true;
  const int NL = a.W.layers;
  const int tid = tid_opaque();
  const int g = tid / ILL_PART_Q, m = tid - g * ILL_PART_Q;
  const bool act = g < NG;
  int64_t* red = (int64_t*)lds;   // [NG][ILL_PART_Q][3]
  constexpr int PSTRIDE = ILL_MAXT * ILL_PART_ROW * 16;   // bytes per producer
  const int off = (t * ILL_PART_ROW + q * ILL_PART_Q + m) * 16;
  const int col = ILL_RED_COLS * q + tid;   // the column of threads tid < ILL_RED_COLS
  if (tid < ILL_RED_COLS) fx_add(acc_ptr(a, H.bank, 0, 0, t) + acc_col(col), fx_word(fx_of(embed1(a.W, H.tok[t], col))));
  for (int l = 0; l < NL; l++) {
    trace_mark(a, ILL_TRL * l);
    const uint32_t tag = tagof_pub(H.epoch, l);
    const __amdgpu_buffer_rsrc_t rs = pub_rsrc(a.part + (size_t)(l & 1) * ILL_NGU * ILL_MAXT * ILL_PART_ROW, ILL_NGU * PSTRIDE);
    int64_t s0 = 0, s1 = 0, s2 = 0;
    auto full = [&]() {
      bool ok = true;
      s0 = s1 = s2 = 0;
      if (act) {
        ill_v4u wv[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
          const int p = g + NG * i;
          wv[i] = (ill_v4u){0u, 0u, 0u, 0u};
          if (p < ILL_NGU) wv[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, opq(off + p * PSTRIDE), 0, ILL_BUF_SC1);
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
          if (g + NG * i < ILL_NGU) {
            ok &= pub_ok(wv[i], tag);
            s0 += fx_of(__uint_as_float(wv[i][0]));
            s1 += fx_of(__uint_as_float(wv[i][1]));
            s2 += fx_of(__uint_as_float(wv[i][2]));
          }
        }
      }
      return ok;
    };
    bool alive;
    if constexpr (ILL_WATCH_RED) {
      // wave 0 watches one word (the first of the segment) of producers 0 .. NG - 1, the
      // others wait at the barrier; its verdict goes through red[0], which the sums
      // overwrite only after the barrier below
      if (tid < 64) {
        const int l64 = tid;
        const int o0 = (t * ILL_PART_ROW + q * ILL_PART_Q) * 16 + min(l64, NG - 1) * PSTRIDE;
        const bool lit = wave_light_p<ILL_POLL_D, ILL_WATCH_SLEEP, ill_v4u>(
            [&](ill_v4u& v) { v = __builtin_amdgcn_raw_buffer_load_b128(rs, opq(o0), 0, ILL_BUF_SC1); },
            [&](const ill_v4u& v) { return pub_ok(v, tag); }, a.ctl, 900 + l);
        if (tid == 0) red[0] = lit;
      }
      lds_barrier();
      alive = red[0] != 0 && wave_wait(full, a.ctl, 900 + l);
    } else {
      alive = wave_wait2([&]() {
        return !act || pub_ok(__builtin_amdgcn_raw_buffer_load_b128(rs, opq(off + g * PSTRIDE), 0, ILL_BUF_SC1), tag);
      }, full, a.ctl, 900 + l);
    }
    if (!__syncthreads_and(alive)) return false;
    trace_mark(a, ILL_TRL * l + 1);
    if (act) {
      red[(g * ILL_PART_Q + m) * 3 + 0] = s0;
      red[(g * ILL_PART_Q + m) * 3 + 1] = s1;
      red[(g * ILL_PART_Q + m) * 3 + 2] = s2;
    }
    __syncthreads();
    bool xa_ok = true;
    if (tid < ILL_RED_COLS) {
      const int mm = tid / 3, i = tid - 3 * (tid / 3);
      int64_t sum = 0;
#pragma unroll
      for (int gg = 0; gg < NG; gg++) sum += red[(gg * ILL_PART_Q + mm) * 3 + i];
      // XA[l] (14 heads and this workgroup's base): long complete when the partials arrive
      const uint64_t* xa = acc_ptr(a, H.bank, l, 0, t) + acc_col(col);
      uint64_t xw = 0;
      xa_ok = wave_wait([&]() {
        xw = aload64(xa);
        return fx_count(xw) == xa_expect<T>(0);
      }, a.ctl, 950 + l);
      sum += fx_value(xw);
      constexpr int64_t NB = ILL_NGU + 1;
      fx_add(acc_ptr(a, H.bank, l, ILL_KIND_XB, t) + acc_col(col), (uint64_t)NB * FX_COUNT + (uint64_t)(sum + NB * FX_BIAS));
      if (l + 1 < NL) fx_add(acc_ptr(a, H.bank, l + 1, 0, t) + acc_col(col), fx_word(sum));
    }
    if (!__syncthreads_and(xa_ok)) return false;
    trace_mark(a, ILL_TRL * l + 10);
    if (a.trace) {
      wait_vm();
      trace_mark(a, ILL_TRL * l + 12);
    }
    __syncthreads();   // red is rewritten by the next layer
    trace_mark(a, ILL_TRL * l + 11);
  }
  return true;
}

// 16-row passes: the partial chunk c (the chunk holding pos, or the one after it) for
// every row at once. Keys and values at positions >= pos are the pass rows on each row's
// path. Scores: the blocks holding cached keys from the cache (all rows), the pass
// positions from one 16 x 16 block SP[t][j] = q_t . k_j over the pass rows j, gathered along
// each row's path. Every score is the MFMA product of the same operands as in a 1-row pass
// at that row's position, and the softmax runs in the same lane layout, so a row's maximum
// and sum match that pass bit for bit. The value operand differs per row, so each row's
// P x V runs on its own operand (the cached values below pos, the table of path values vq
// above it), with the 1-row pass's instruction sequence. Wave w finishes the one row of
// rows w and w + 8 that belongs to its workgroup (rows rlo .. rhi - 1): its statistics and
// output go to A.pm / A.pl / A.po[c - ns].
// vq (stage + ILL_ST_VPT): [row t][dim][24] f16, the values at positions 8 (pos / 8) + q,
// q < 24 (a range holding pos .. pos + 15): path row values at depths 0 .. depth(t), else 0.
template <int T>
__device__ __forceinline__ void part_eval16(const PassHdr& H, AttLds<T>& A, const uint8_t* stage, const KVFrag& f, int c,
                                            bool cache, const v8h qa[2][2], int rlo, int rhi) {
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int pos = H.pos, nrows = H.nrows, ns = pos >> 6;
  const uint4 zz = make_uint4(0, 0, 0, 0);
  float* pb = att_pbuf<T>(A, w);
  // SP: lane (kg, n) holds q_t . k_n for rows t = 4 kg + j
  v4f sp = {0.f, 0.f, 0.f, 0.f};
  {
    const int kr = arow<T>(n);   // pass rows beyond T: copies (their columns are never gathered)
    const v8h k0 = u4_to_v8h(*(const uint4*)&A.k[kr][8 * kg]), k1 = u4_to_v8h(*(const uint4*)&A.k[kr][32 + 8 * kg]);
    sp = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][0], k0, sp, 0, 0, 0);
    sp = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][1], k0, sp, 0, 0, 0);
    sp = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][0], k1, sp, 0, 0, 0);
    sp = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][1], k1, sp, 0, 0, 0);
  }
  // The one row this wave finishes (rows w and w + 8 that belong to this workgroup: at
  // most one), and its place j0 = t0 % 4 in the lanes' row blocks. The softmax runs for
  // rows 4 kg + j0 only (t0 among them); the other rows' P stays unwritten, and their P.V
  // outputs are not used.
  int t0 = -1;
#pragma unroll
  for (int r = 0; r < 2; r++)
    if (w + ILL_WAVES * r >= rlo && w + ILL_WAVES * r < rhi) t0 = w + ILL_WAVES * r;
  if (t0 < 0) return;
  const int j0 = t0 & 3, tr = 4 * kg + j0;
  const int Lr = tr < nrows ? pos + H.depth[tr] + 1 : 0;   // L of this lane's row (0: no row)
  float sc[4];
#pragma unroll
  for (int b = 0; b < 4; b++) {
    const int vp = 64 * c + 16 * b + n;
    v4f s = {0.f, 0.f, 0.f, 0.f};
    if (cache && 64 * c + 16 * b < pos) {   // wave-uniform: the block holds cached keys
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][0], u4_to_v8h(f.k[b][0]), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[0][1], u4_to_v8h(f.k[b][0]), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][0], u4_to_v8h(f.k[b][1]), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[1][1], u4_to_v8h(f.k[b][1]), s, 0, 0, 0);
    }
    const int dd = min(max(vp - pos, 0), 15);   // depth of a pass position
    const int src = (lane & 48) | H.prow[tr][dd];
    const float g = __shfl(j0 == 0 ? sp[0] : j0 == 1 ? sp[1] : j0 == 2 ? sp[2] : sp[3], src, 64);
    const float sv = j0 == 0 ? s[0] : j0 == 1 ? s[1] : j0 == 2 ? s[2] : s[3];
    sc[b] = vp < pos ? sv : (vp < Lr ? g : -INFINITY);
  }
  float mx, ls;
  {
    const float m = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mx = gmax<16>(m);
    float sum = 0.f;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      sc[b] = att_exp(sc[b] - mx);
      sum += sc[b];
    }
    ls = gsum<16>(sum);
  }
#pragma unroll
  for (int b = 0; b < 4; b++)
    if (tr < T) pb[tr * 64 + 16 * b + n] = sc[b];
  wave_lds_sync();
  v8h ph[2], pl[2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float p = pb[arow<T>(n) * 64 + 32 * ks + 8 * kg + i];
      const _Float16 hi = (_Float16)p;
      ph[ks][i] = hi;
      pl[ks][i] = (_Float16)(p - (float)hi);
    }
  }
  wave_lds_sync();
  const uint4* vq = (const uint4*)(stage + ILL_ST_VPT);
  {
    const int t = t0, j = j0;
    const int Lt = pos + H.depth[t] + 1;
    if (Lt <= 64 * c) return;   // wave-uniform: no position of the chunk is on the row's path
    if (kg == (t >> 2) && n == 0) {
      A.pm[c - ns][t] = mx;
      A.pl[c - ns][t] = ls;
    }
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
      const int dim = 16 * nb + n;
      v8h vv[2];
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const int p0 = 64 * c + 32 * ks + 8 * kg;   // this lane's first position
        const int sl = (p0 >> 3) - (pos >> 3);      // its 8-group in vq
        uint4 u = cache ? f.v[nb][ks] : zz;
        if (sl >= 0 && sl < 3) {
          // halves below pos (the first pos - p0 < 8) from the cache, the rest from vq
          const uint4 x = vq[((size_t)t * 64 + dim) * 3 + sl];
          const int nc = pos - p0;
          auto mg = [&](uint32_t uc, uint32_t xt, int k) {
            return 2 * k + 1 < nc ? uc : (2 * k >= nc ? xt : ((uc & 0xffffu) | (xt & 0xffff0000u)));
          };
          u = make_uint4(mg(u.x, x.x, 0), mg(u.y, x.y, 1), mg(u.z, x.z, 2), mg(u.w, x.w, 3));
        }
        vv[ks] = u4_to_v8h(u);
      }
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[0], vv[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[0], vv[0], acc, 0, 0, 0);
      // positions 32 .. 63 all beyond the row's path hold p = 0: skipped, as the 1-row pass does
      if (64 * c + 32 < Lt) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[1], vv[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[1], vv[1], acc, 0, 0, 0);
      }
      if (kg == (t >> 2)) A.po[c - ns][t][dim] = j == 0 ? acc[0] : j == 1 ? acc[1] : j == 2 ? acc[2] : acc[3];
    }
  }
}

// Chunk of the partial (chunk, row) pair number `idx` (pairs run over chunks c >= ns, then
// rows t with L(t) > 64 c), or -1. (At T = 1 there is one pair: chunk ns, row 0. This form,
// rather than the equivalent sj == ns test, measured 1.5% faster per step: it changes how
// the compiler schedules the first fetch.)
__device__ __forceinline__ int att_pair_chunk(const PassHdr& H, int ns, int cmax, int idx) {
  int k = 0;
  for (int c = ns; c <= cmax; c++)
    for (int t = 0; t < H.nrows; t++)
      if (H.pos + H.depth[t] + 1 > 64 * c) {
        if (k == idx) return c;
        k++;
      }
  return -1;
}

template <int T>
__device__ __forceinline__ bool role_att(const IllPassArgs& a, const PassHdr& H, AttLds<T>& A, int l, int h, int half, uint8_t* stage) {
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int g = h / 7;
  const IllLayerW Lc = layer_ptrs(a.L, l);
  const IllLayerW& L = T == 1 ? a.L[l] : Lc;
  constexpr int RPL = T >= 4 ? 4 : T;
  const int nrows = H.nrows;
  const int pos = H.pos;
  // 16-row passes split the rows over two workgroups per head (half 0: rows 0-7, half 1:
  // rows 8-15); both compute every row's q, k and v (the tiles are 16 rows wide anyway) and
  // the shared chunks, and each finishes its own rows: path values, the partial chunk's
  // P·V, the combine and the O contributions
  const int rlo = ill_pub<T>() ? 8 * half : 0, rhi = ill_pub<T>() ? min(nrows, rlo + 8) : nrows;
  // QKV epilogue constants (independent of the input): bias and RoPE (cos, sin) per row
  const int nt = qkv_nt<T>(w), lt0 = qkv_lt0<T>(w);
  const int bw = lt0 >> 1, hf1 = nt == 1 ? (lt0 & 1) : 0;   // block; a single tile's half
  const int d = (att_block(h, nt > 0 ? bw : 0) & 1) * 16 + n;
  float bias0 = 0.f, bias1 = 0.f;
  float2 rope[4] = {};
  if (nt > 0) {
    const int b = att_block(h, bw);
    bias0 = gld(L.bqkv + 32 * b + 16 * hf1 + n);
    bias1 = gld(L.bqkv + 32 * b + 16 + n);
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t < nrows) rope[j] = gld(a.rope + (pos + H.depth[t]) * 32 + d);
    }
  }
  // ---- attention work of this wave's slot sj: shared chunks sj, sj + 8, ... < ns, then
  // the partial pairs idx = sj - ns (mod 8), + 8, ...
  const int sj = att_slot<T>(w);
  int maxL = 0;
  for (int t = 0; t < nrows; t++) maxL = max(maxL, pos + H.depth[t] + 1);
  const int ns = pos >> 6, cmax = (maxL - 1) >> 6;
  const uint16_t* kbase = a.kc + ((size_t)l * ILL_NKV + g) * a.maxctx * 64;
  const uint16_t* vbase = a.vt + ((size_t)l * ILL_NKV + g) * (a.maxctx / 64) * 64 * 64;
  // Waves without a shared chunk: at T = 1 the wave of the partial pair fetches chunk ns; in
  // 16-row passes every wave evaluates chunk ns, which needs the cache if it holds positions
  // below pos.
  const int cfirst = sj < ns ? sj : (T == 1 ? att_pair_chunk(H, ns, cmax, (sj - ns) & 7) : (64 * ns < pos ? ns : -1));
  KVFrag f;
  int fc = -1;   // cache chunk held in f
  // The slot's first chunk streams in while the input is awaited: cache positions below pos
  // were written by earlier passes, and the positions of this pass are taken from LDS.
  // (Waves without attention work issue nothing: a fetch costs the CU's memory-issue
  // bandwidth.)
  if (cfirst >= 0) {
    kv_fetch(kbase, vbase, cfirst, lane, f);
    fc = cfirst;
  }
  // ---- input x_l: embedding (layer 0) or the completed accumulator XB[l-1]
  bool ok;
  float rs[4];   // RMSNorm scale of this lane's rows
  if constexpr (ill_pub<T>()) ok = pub_read<T>(pub_ptr(a, 1, l, 0), tagof_pub(H.epoch, l), nrows, A.u.prep, a.ctl, 100 + l, a, rs, ILL_TRL * l + 15);
  else if (l == 0) ok = prep896<T>(SrcEmbed{a.W, H.tok}, L.ln1, nrows, A.u.prep, a.ctl, 100 + l, a, rs);
  else ok = prep896<T>(SrcXB<T>{acc_ptr(a, H.bank, l - 1, ILL_KIND_XB, 0)}, L.ln1, nrows, A.u.prep, a.ctl, 100 + l, a, rs, ILL_TRL * l + 15);
  if (!ok) return false;
  trace_mark(a, ILL_TRL * l + 1);
  // ---- q_h, k_g, v_g rows (the wave's row tiles, see qkv_nt)
  float acc0[4] = {0.f, 0.f, 0.f, 0.f}, acc1[4] = {0.f, 0.f, 0.f, 0.f};
  wait_vm();   // every wave: its staged weights, the epilogue constants and its first chunk
  // pin the epilogue constants here: a load sunk to its use would be waited for in the
  // middle of the attention work
  asm volatile("" ::"v"(bias0), "v"(bias1));
#pragma unroll
  for (int j = 0; j < RPL; j++) asm volatile("" ::"v"(rope[j].x), "v"(rope[j].y));
  trace_mark(a, ILL_TRL * l + 2);
  const uint8_t* st = stage + lt0 * ILL_ST_TILE;
  if constexpr (T == 1) {
    float accs[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    if (nt == 2) q4_tiles896_lds<T, 2>(st, ILL_ST_TILE, A.u.prep, lane, accs);
    else q4_tiles896_lds<T, 1>(st, ILL_ST_TILE, A.u.prep, lane, accs);
    acc0[0] = accs[0][0];
    acc1[0] = accs[1][0];
    trace_mark(a, ILL_TRL * l + 3);
  } else if (nt == 2) {   // two tiles sharing each group's activation reads
    float accs[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    q4_tiles896_lds<T, 2>(st, ILL_ST_TILE, A.u.prep, lane, accs);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      acc0[j] = accs[0][j];
      acc1[j] = accs[1][j];
    }
    trace_mark(a, ILL_TRL * l + 3);
  } else {
    q4_tile896_lds<T>(st, st + ILL_KST * 1024, A.u.prep, lane, acc0);
    trace_mark(a, ILL_TRL * l + 3);
  }
  if (nt == 1) {   // one half of a v block: no RoPE
    const int dim = d + 32 * hf1;
    const bool writer = (h % 7) == 0 && half == 0;   // one workgroup per group writes the V cache
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t >= nrows) continue;
      const uint32_t h0 = f2h_sat(acc0[j] * rs[j] + bias0);
      A.v[t][dim] = (uint16_t)h0;
      if (writer) {
        const int slot = pos + t;
        uint16_t* vb = a.vt + (((size_t)l * ILL_NKV + g) * (a.maxctx / 64) + slot / 64) * 64 * 64;
        gst(vb + dim * 64 + (slot & 63), (uint16_t)h0);
      }
    }
  } else if (nt == 2) {
    const int b = att_block(h, bw);
    const int head = b >> 1;
    const bool writer = (h % 7) == 0 && half == 0;   // one workgroup per group writes the K/V cache
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t >= nrows) continue;
      float x0 = acc0[j] * rs[j] + bias0, x1 = acc1[j] * rs[j] + bias1;
      if (head < ILL_NH + ILL_NKV) {
        const float2 cs = rope[j];
        const float r0 = x0 * cs.x - x1 * cs.y;
        const float r1 = x1 * cs.x + x0 * cs.y;
        x0 = r0;
        x1 = r1;
      }
      const int slot = pos + t;
      if (head < ILL_NH) {
        A.q[t][d] = x0;
        A.q[t][d + 32] = x1;
      } else if (head < ILL_NH + ILL_NKV) {
        const uint32_t h0 = f2h(x0), h1 = f2h(x1);
        A.k[t][d] = (uint16_t)h0;
        A.k[t][d + 32] = (uint16_t)h1;
        if (writer) {
          uint16_t* kr = a.kc + (((size_t)l * ILL_NKV + g) * a.maxctx + slot) * 64;
          gst(kr + d, (uint16_t)h0);
          gst(kr + d + 32, (uint16_t)h1);
        }
      } else {
        const uint32_t h0 = f2h_sat(x0), h1 = f2h_sat(x1);
        A.v[t][d] = (uint16_t)h0;
        A.v[t][d + 32] = (uint16_t)h1;
        if (writer) {
          uint16_t* vb = a.vt + (((size_t)l * ILL_NKV + g) * (a.maxctx / 64) + slot / 64) * 64 * 64;
          gst(vb + d * 64 + (slot & 63), (uint16_t)h0);
          gst(vb + (d + 32) * 64 + (slot & 63), (uint16_t)h1);
        }
      }
    }
  }
  lds_barrier();
  trace_mark(a, ILL_TRL * l + 4);
  if (T != 1) att_stage_o<T>(L, h, w, lane, stage);   // O weights stream in while attention runs
  if constexpr (T > 1) {   // path values of the pass rows at positions 8 (pos / 8) + q, q < 24 (part_eval16)
    uint4* vq = (uint4*)(stage + ILL_ST_VPT);
    const int d0 = 8 * (pos >> 3) - pos;   // depth of q = 0 (-7 .. 0)
    static_assert(T * 32 <= ILL_WG_THREADS, "one thread per (row, dim pair)");
    const int t1 = min(tid >> 5, T - 1), dp = tid & 31;   // row t1, dims 2 dp and 2 dp + 1
    const int dep = (tid >> 5) >= rlo && (tid >> 5) < rhi ? H.depth[t1] : -1;   // (rows of this workgroup)
    uint32_t e[24];   // both dims' values (low half: dim 2 dp)
#pragma unroll
    for (int q = 0; q < 24; q++) {
      const int dd = d0 + q;
      e[q] = dd >= 0 && dd <= dep ? *(const uint32_t*)&A.v[min(H.prow[t1][min(dd, 15)], T - 1)][2 * dp] : 0u;
    }
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      uint32_t h[24];
#pragma unroll
      for (int q = 0; q < 24; q++) h[q] = hf ? e[q] >> 16 : e[q] & 0xffffu;
#pragma unroll
      for (int s3 = 0; s3 < 3; s3++)
        if ((tid >> 5) < T) vq[(t1 * 64 + 2 * dp + hf) * 3 + s3] = make_uint4(h[8 * s3] | (h[8 * s3 + 1] << 16), h[8 * s3 + 2] | (h[8 * s3 + 3] << 16),
                                                         h[8 * s3 + 4] | (h[8 * s3 + 5] << 16), h[8 * s3 + 6] | (h[8 * s3 + 7] << 16));
    }
    lds_barrier();
  }
  trace_mark(a, ILL_TRL * l + 5);
  // ---- attention for head h
  v8h qa[2][2];   // [ks][hi/lo], lane (kg, m = row), dims 32 ks + 8 kg + i, q * 0.125
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float v = A.q[arow<T>(n)][32 * ks + 8 * kg + i] * 0.125f;
      const _Float16 hi = (_Float16)v;
      qa[ks][0][i] = hi;
      qa[ks][1][i] = (_Float16)(v - (float)hi);
    }
  }
  float M[4], Lw[4], O[4][4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    M[j] = -INFINITY;
    Lw[j] = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; nb++) O[nb][j] = 0.f;
  }
  auto fold = [&](const float mx[4], const float ls[4], const float o[4][4]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const AttScale k = att_scale(M[j], mx[j]);
#pragma unroll
      for (int nb = 0; nb < 4; nb++) O[nb][j] = att_fold(O[nb][j], o[nb][j], k);
      Lw[j] = att_fold(Lw[j], ls[j], k);
      M[j] = k.mn;
    }
  };
  for (int c = sj; c < ns; c += ILL_WAVES) {
    if (c != fc) {
      kv_fetch(kbase, vbase, c, lane, f);
      fc = c;
    }
    float mx[4], ls[4], o[4][4];
    chunk_eval<T>(H, A, stage, f, c, false, 0, qa, mx, ls, o);
    fold(mx, ls, o);
  }
  if constexpr (T == 1) {
    // the one partial pair (chunk ns, row 0) belongs to slot ns % 8, whose wave folds it
    // into the slot state after the slot's shared chunks, as the combine would
    if (sj == (ns & 7)) {
      if (ns != fc) {
        kv_fetch(kbase, vbase, ns, lane, f);
        fc = ns;
      }
      float mx[4], ls[4], o[4][4];
      chunk_eval<T>(H, A, stage, f, ns, true, 0, qa, mx, ls, o);
      fold(mx, ls, o);
    }
  } else {
    for (int c = ns; c <= cmax; c++) {
      const bool cache = 64 * c < pos;
      if (cache && c != fc) {
        kv_fetch(kbase, vbase, c, lane, f);
        fc = c;
      }
      part_eval16<T>(H, A, stage, f, c, cache, qa, rlo, rhi);
    }
  }
  trace_mark(a, ILL_TRL * l + 6);
  if (T > 1) lds_barrier();   // LDS: the P region becomes the combine region
  trace_mark(a, ILL_TRL * l + 13);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int t = 4 * kg + j;
    if (t < T) {
      if (n == 0) {
        A.u.c.cm[sj][t] = M[j];
        A.u.c.cl[sj][t] = Lw[j];
      }
#pragma unroll
      for (int nb = 0; nb < 4; nb++) A.u.c.co[sj][t][16 * nb + n] = O[nb][j];
    }
  }
  lds_barrier();
  trace_mark(a, ILL_TRL * l + 14);
  // combine: slot states (+ the partial chunks of each slot, in chunk order), then across
  // slots against the global maximum; row t by wave t % 8, one dim per lane, then the row
  // is coded as the A operand of the O projection (one quant group: head h's columns)
  for (int t = w; t < T; t += ILL_WAVES) {
    if (t < rlo || t >= rhi) {   // not this workgroup's row (or not live): coded as zeros
      if (lane < 4) {
        A.ahi[lane * T + t] = make_uint4(0, 0, 0, 0);
        A.alo[lane * T + t] = make_uint4(0, 0, 0, 0);
      }
      continue;
    }
    const int dim = lane;
    const int Lt = pos + H.depth[t] + 1;
    float sm[ILL_WAVES], sl[ILL_WAVES], so[ILL_WAVES];
#pragma unroll
    for (int ww = 0; ww < ILL_WAVES; ww++) {
      sm[ww] = A.u.c.cm[ww][t];
      sl[ww] = A.u.c.cl[ww][t];
      so[ww] = A.u.c.co[ww][t][dim];
#pragma unroll
      for (int ci = 0; ci < (T > 1 ? 2 : 0); ci++) {   // at T = 1 the slot's wave folded it
        const int c = ns + ci;
        if ((c & 7) == ww && c <= cmax && Lt > 64 * c) {
          const AttScale k = att_scale(sm[ww], A.pm[ci][t]);
          so[ww] = att_fold(so[ww], A.po[ci][t][dim], k);
          sl[ww] = att_fold(sl[ww], A.pl[ci][t], k);
          sm[ww] = k.mn;
        }
      }
    }
    float m = sm[0];
#pragma unroll
    for (int ww = 1; ww < ILL_WAVES; ww++) m = fmaxf(m, sm[ww]);
    float sum = 0.f, o = 0.f;
#pragma unroll
    for (int ww = 0; ww < ILL_WAVES; ww++) {
      const float e = att_exp(sm[ww] - m);
      sum = sum + sl[ww] * e;
      o = o + so[ww] * e;
    }
    quant_row64<T>(o / sum, t, A.ahi, A.alo, A.dsc, lane);
  }
  trace_mark(a, ILL_TRL * l + 7);
  lds_barrier();
  trace_mark(a, ILL_TRL * l + 8);
  wait_vm();   // this wave's staged O tiles
  trace_mark(a, ILL_TRL * l + 9);
  split_gemv<T>(stage + ill_st_o(T) + w * ILL_ST_SPLIT, A.ahi, A.alo, A.dsc, lane, rhi,
                acc_ptr(a, H.bank, l, h % xa_copies<T>(), 0) + acc_col(16 * 7 * w), rlo);
  trace_mark(a, ILL_TRL * l + 10);
  if (a.trace) {   // traced runs only: when this wave's contributions have landed
    wait_vm();
    trace_mark(a, ILL_TRL * l + 12);
  }
  return true;
}

// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void gud_stage(const IllLayerW& L, int ub, int w, int lane, uint8_t* stage) {
  const int tile = ub * 8 + w;
  uint8_t* d = stage + w * ILL_ST_GU;
  wave_copy_to_lds(L.wgu + (size_t)tile * ILL_KST * 1024, d, ILL_KST * 1024, lane);
  wave_copy_to_lds((const uint8_t*)(L.sgu + tile * ILL_KST * 32), d + ILL_KST * 1024, ILL_KST * 128, lane);
  split_stage(L.wd + (size_t)ub * ILL_NOT * 512, L.sd + ub * ILL_NOT * 16, w, lane, stage + ILL_ST_DOWN0 + w * ILL_ST_SPLIT);
}

template <int T>
__device__ __forceinline__ bool role_gud(const IllPassArgs& a, const PassHdr& H, GudLds<T>& G, int l, int ub, uint8_t* stage) {
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const IllLayerW Lc = layer_ptrs(a.L, l);
  const IllLayerW& L = T == 1 ? a.L[l] : Lc;
  const int nrows = H.nrows;
  constexpr int RPL = T >= 4 ? 4 : T;
  float rs[4];   // RMSNorm scale of this lane's rows
  bool ok;
  if constexpr (ill_pub<T>()) ok = pub_read<T>(pub_ptr(a, 0, l, 0), tagof_pub(H.epoch, l), nrows, G.prep, a.ctl, 400 + l, a, rs, ILL_TRL * l + 6);
  else ok = prep896<T>(SrcXA<T>{acc_ptr(a, H.bank, l, 0, 0)}, L.ln2, nrows, G.prep, a.ctl, 400 + l, a, rs, ILL_TRL * l + 6);
  if (!ok) return false;
  trace_mark(a, ILL_TRL * l + 1);
  {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    wait_vm();   // this wave's staged gate/up tile and down tiles
    trace_mark(a, ILL_TRL * l + 2);
    const uint8_t* sg = stage + w * ILL_ST_GU;
    q4_tile896_lds<T>(sg, sg + ILL_KST * 1024, G.prep, lane, acc);
    trace_mark(a, ILL_TRL * l + 3);
#pragma unroll
    for (int j = 0; j < RPL; j++) {
      const int t = 4 * kg + j;
      if (t < T) G.gu[w][t][n] = acc[j] * rs[j];
    }
  }
  lds_barrier();
  trace_mark(a, ILL_TRL * l + 4);
  if constexpr (T == 1) {
    // every wave codes the SiLU row itself (the arithmetic one wave would run for all) into
    // its own LDS copy, so its down projection waits for no other wave
    const int gi = lane >> 4, nn = lane & 15;
    const float gv = G.gu[gi][0][nn], up = G.gu[4 + gi][0][nn];
    uint4* ah = G.wahi + 4 * w;
    uint4* al = G.walo + 4 * w;
    float2* ds = G.wdsc + w;
    quant_row64<1>(gv / (1.0f + expf(-gv)) * up, 0, ah, al, ds, lane);
    wave_lds_sync();
    trace_mark(a, ILL_TRL * l + 5);
    split_gemv<T>(stage + ILL_ST_DOWN0 + w * ILL_ST_SPLIT, ah, al, ds, lane, nrows,
                  acc_ptr(a, H.bank, l, ILL_KIND_XB + ub % xb_copies<T>(), 0) + acc_col(16 * 7 * w));
    trace_mark(a, ILL_TRL * l + 10);
    if (a.trace) {   // traced runs only: when this wave's contributions have landed
      wait_vm();
      trace_mark(a, ILL_TRL * l + 12);
    }
    return true;
  }
  // SiLU(gate) * up for the block's 64 units; each row coded as one 64-wide group
  for (int t = w; t < T; t += ILL_WAVES) {
    if (t < nrows) {
      const int gi = lane >> 4, nn = lane & 15;
      const float gv = G.gu[gi][t][nn], up = G.gu[4 + gi][t][nn];
      quant_row64<T>(gv / (1.0f + expf(-gv)) * up, t, G.ahi, G.alo, G.dsc, lane);
    } else if (lane < 4) {
      G.ahi[lane * T + t] = make_uint4(0, 0, 0, 0);
      G.alo[lane * T + t] = make_uint4(0, 0, 0, 0);
    }
  }
  lds_barrier();
  trace_mark(a, ILL_TRL * l + 5);
  if constexpr (ill_pub<T>()) {
    // 16-row passes: the partial leaves as plain checked words, and the REDUCE workgroups
    // make one accumulator contribution per word out of the 76 partials (the atomics of 76
    // workgroups x 16 rows would queue at the memory side for several microseconds)
    float y[7][4];
    split_outputs<T>(stage + ILL_ST_DOWN0 + w * ILL_ST_SPLIT, G.ahi, G.alo, G.dsc, lane, y);
    float* yt = (float*)stage;   // [16][896]: the gate/up stage, free after the gate/up GEMM
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int t = 4 * kg + j;
#pragma unroll
      for (int k = 0; k < 7; k++)
        if (t < nrows) yt[t * ILL_H + 112 * w + 16 * k + n] = y[k][j];
    }
    lds_barrier();
    part_write(a, H.epoch, l, ub, yt, nrows);
  } else {
    split_gemv<T>(stage + ILL_ST_DOWN0 + w * ILL_ST_SPLIT, G.ahi, G.alo, G.dsc, lane, nrows,
                  acc_ptr(a, H.bank, l, ILL_KIND_XB + ub % xb_copies<T>(), 0) + acc_col(16 * 7 * w));
  }
  trace_mark(a, ILL_TRL * l + 10);
  if (a.trace) {   // traced runs only: when this wave's contributions have landed
    wait_vm();
    trace_mark(a, ILL_TRL * l + 12);
  }
  return true;
}

// ---------------------------------------------------------------------------------------
// BASE (one workgroup): the residual itself is the last contributor of each accumulator.
// It adds x_l (the embedding at layer 0, else the completed XB[l-1]) into XA[l], then the
// completed XA[l] into XB[l]. It runs beside the ATT and GUD work of the same layer, so
// the copies stay off the critical path.
template <int T>
__device__ __forceinline__ bool role_base(const IllPassArgs& a, const PassHdr& H, int l) {
  const int tid = tid_opaque();
  constexpr int PER = (T * ILL_H + ILL_WG_THREADS - 1) / ILL_WG_THREADS;
  const int n = H.nrows * ILL_H;
  auto at = [](int i) { return (size_t)(i / ILL_H) * ILL_ACC_ROW + acc_col(i % ILL_H); };   // element i = row * 896 + column
  auto wait_full = [&](const uint64_t* src, int expect, int code) {
    return wg_wait([&]() {
      bool r = true;
#pragma unroll
      for (int k = 0; k < PER; k++) {
        const int i = tid + k * ILL_WG_THREADS;
        if (i < n) r &= fx_count(aload64(src + at(i))) == expect;
      }
      return r;
    }, a.ctl, code);
  };
  uint64_t* xa = acc_ptr(a, H.bank, l, 0, 0);
  uint64_t* xb = acc_ptr(a, H.bank, l, ILL_KIND_XB, 0);
  if (l == 0) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int i = tid + k * ILL_WG_THREADS;
      if (i < n) fx_add(xa + at(i), fx_word(fx_of(embed1(a.W, H.tok[i / ILL_H], i % ILL_H))));
    }
  } else {
    const uint64_t* prev = acc_ptr(a, H.bank, l - 1, ILL_KIND_XB, 0);
#pragma unroll
    for (int c = 0; c < xb_copies<T>(); c++)
      if (!wait_full(prev + (size_t)c * 16 * ILL_ACC_ROW, xb_expect<T>(c), 800 + l)) return false;
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int i = tid + k * ILL_WG_THREADS;
      if (i < n) {
        int64_t sum = 0;
#pragma unroll
        for (int c = 0; c < xb_copies<T>(); c++) sum += fx_value(aload64(prev + (size_t)c * 16 * ILL_ACC_ROW + at(i)));
        fx_add(xa + at(i), fx_word(sum));
      }
    }
  }
#pragma unroll
  for (int c = 0; c < xa_copies<T>(); c++)
    if (!wait_full(xa + (size_t)c * 16 * ILL_ACC_ROW, xa_expect<T>(c), 850 + l)) return false;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int i = tid + k * ILL_WG_THREADS;
    if (i < n) {
      int64_t sum = 0;
#pragma unroll
      for (int c = 0; c < xa_copies<T>(); c++) sum += fx_value(aload64(xa + (size_t)c * 16 * ILL_ACC_ROW + at(i)));
      fx_add(xb + at(i), fx_word(sum));
    }
  }
  return true;
}

// ---------------------------------------------------------------------------------------
// PREP (16-row passes, one workgroup per row t < nrows): the published codings of row t,
// layer by layer, in the order the pass needs them: the ATT input x_l (the embedding at
// layer 0, else the completed XB[l-1]) under ln1, then the GUD input XA[l] under ln2, and
// after the last layer the final-norm input of the lm_head.
template <int T>
__device__ __forceinline__ bool role_prep(const IllPassArgs& a, const PassHdr& H, PrepLds<1>& P, int t) {
  const int NL = a.W.layers;
  float rs[4];
  for (int l = 0; l <= NL; l++) {
    const float* gam = l < NL ? a.L[l].ln1 : a.W.fnorm;
    bool ok;
    const int tr = l < NL ? ILL_TRL * l : -1;   // trace: 1/2 input seen / coded, 3 published, 5-7 the same for XA
    if (l == 0) ok = prep896<1>(SrcEmbed{a.W, H.tok + t}, gam, 1, P, a.ctl, 700, a, rs, tr < 0 ? -1 : tr + 1);
    else ok = prep896<1>(SrcXB<T>{acc_ptr(a, H.bank, l - 1, ILL_KIND_XB, t)}, gam, 1, P, a.ctl, 700 + l, a, rs, tr < 0 ? -1 : tr + 1);
    if (!ok) return false;
    pub_write(P, rs[0], pub_ptr(a, 1, l, t), tagof_pub(H.epoch, l));
    lds_barrier();   // the coding is read out before the next one is written
    if (l == NL) break;
    trace_mark(a, tr + 3);
    if (!prep896<1>(SrcXA<T>{acc_ptr(a, H.bank, l, 0, t)}, a.L[l].ln2, 1, P, a.ctl, 750 + l, a, rs, tr + 5)) return false;
    pub_write(P, rs[0], pub_ptr(a, 0, l, t), tagof_pub(H.epoch, l));
    lds_barrier();
    trace_mark(a, tr + 7);
  }
  return true;
}

// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void amax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

// The lm_head over the final RMSNorm (tied embedding rows, 16-row tiles), with the per-row
// argmax partials published for the commit. In 1-row passes the workgroups with no layer
// role (ILL_R_IDLE0..255) copy ILL_LMH_PRE tiles each into their free LDS stage while they
// wait for the last layer, and those tiles come off the stream the other workgroups share
// after the last edge (the argmax and the logits do not depend on which workgroup holds a
// tile; the products run the same code on either source).
template <int T>
__device__ __forceinline__ bool role_lmh(const IllPassArgs& a, const PassHdr& H, LmhLds<T>& Lm, uint8_t* stage) {
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int kg = lane >> 4, n = lane & 15;
  const int NL = a.W.layers;
  const uint32_t tag = tagof_lmh(H.epoch);
  const int V = a.W.vocab, ntiles = V >> 4;
  const int wg = blockIdx.x;
  float bv[4];
  int bi[4];
#pragma unroll
  for (int j = 0; j < 4; j++) { bv[j] = -INFINITY; bi[j] = 0x7fffffff; }
  static_assert(ILL_LMH_PRE == 2 * ILL_WAVES && ILL_LMH_PRE * ILL_ST_TILE <= ill_stage_bytes(1), "two tiles per wave");
  const bool pre = T == 1 && wg >= ILL_R_IDLE0;
  const int npre = T == 1 ? (ILL_WG - ILL_R_IDLE0) * ILL_LMH_PRE : 0;   // tiles 0 .. npre-1 staged
  const int p0 = (wg - ILL_R_IDLE0) * ILL_LMH_PRE + 2 * w;              // this wave's staged pair
  if (H.lmhn > 0) {
    if (pre) {
#pragma unroll
      for (int i = 0; i < 2; i++) {
        if (p0 + i >= ntiles) continue;
        uint8_t* d = stage + (2 * w + i) * ILL_ST_TILE;
        wave_copy_to_lds(a.W.wemb + (size_t)(p0 + i) * ILL_KST * 1024, d, ILL_KST * 1024, lane);
        wave_copy_to_lds((const uint8_t*)(a.W.semb + (size_t)(p0 + i) * ILL_KST * 32), d + ILL_KST * 1024, ILL_KST * 128, lane);
      }
    }
    int tile = npre + wg + ILL_WG * w;
    Q4Tile cur;
    if (tile < ntiles) q4_load(cur, a.W.wemb + (size_t)tile * ILL_KST * 1024, a.W.semb + (size_t)tile * ILL_KST * 32, lane);
    float rs[4];   // final-norm scale of this lane's rows
    bool ok;
    if constexpr (ill_pub<T>()) ok = pub_read<T>(pub_ptr(a, 1, NL, 0), tagof_pub(H.epoch, NL), H.nrows, Lm.prep, a.ctl, 600, a, rs);
    else ok = prep896<T>(SrcXB<T>{acc_ptr(a, H.bank, NL - 1, ILL_KIND_XB, 0)}, a.W.fnorm, H.nrows, Lm.prep, a.ctl, 600, a, rs);
    if (!ok) return false;
    trace_mark(a, ILL_TR_TAIL + 1);
    constexpr int RPL = T >= 4 ? 4 : T;
    if (pre) {
      wait_vm();   // the staged tiles (copied long before; also the first streamed tile)
      float acc2[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      q4_tiles896_lds<T, 2>(stage + 2 * w * ILL_ST_TILE, ILL_ST_TILE, Lm.prep, lane, acc2);
#pragma unroll
      for (int i = 0; i < 2; i++) {
        if (p0 + i >= ntiles) continue;
        const int idx = 16 * (p0 + i) + n;
#pragma unroll
        for (int j = 0; j < RPL; j++) acc2[i][j] *= rs[j];
#pragma unroll
        for (int j = 0; j < RPL; j++) {
          const int t = 4 * kg + j;
          if (t >= H.lmh0 && t < H.lmh0 + H.lmhn) {
            if (H.wlog) gst(a.logits + (size_t)t * V + idx, acc2[i][j]);
            amax_merge(bv[j], bi[j], acc2[i][j], idx);
          }
        }
      }
    }
    while (tile < ntiles) {
      const int nxt = tile + ILL_WG * ILL_WAVES;
      Q4Tile nx;
      if (nxt < ntiles) q4_load(nx, a.W.wemb + (size_t)nxt * ILL_KST * 1024, a.W.semb + (size_t)nxt * ILL_KST * 32, lane);
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      q4_tile896<T>(cur, Lm.prep, lane, acc);
      const int idx = 16 * tile + n;
#pragma unroll
      for (int j = 0; j < RPL; j++) acc[j] *= rs[j];
#pragma unroll
      for (int j = 0; j < RPL; j++) {
        const int t = 4 * kg + j;
        if (t >= H.lmh0 && t < H.lmh0 + H.lmhn) {
          if (H.wlog) gst(a.logits + (size_t)t * V + idx, acc[j]);
          amax_merge(bv[j], bi[j], acc[j], idx);
        }
      }
      cur = nx;
      tile = nxt;
    }
  }
  constexpr int RPL = T >= 4 ? 4 : T;   // rows per lane: at T = 1 only j = 0 holds a row
#pragma unroll
  for (int j = 0; j < RPL; j++) {
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
  return true;
}

// Zero this workgroup's share of the other accumulator bank (used by the previous pass,
// next used by the following pass).
__device__ __forceinline__ void zero_other_bank(const IllPassArgs& a, const PassHdr& H) {
  if (H.zrows <= 0) return;
  const int NL = a.W.layers;
  const size_t per_row = ILL_H;
  const int other = H.bank ^ 1;
  const size_t nrow_total = (size_t)NL * ILL_NKIND * H.zrows;   // (layer, kind, row) triples
  const size_t total = nrow_total * per_row;
  const size_t chunk = (total + ILL_WG - 1) / ILL_WG;
  const size_t lo = (size_t)blockIdx.x * chunk, hi = min(total, lo + chunk);
  for (size_t i = lo + tid_opaque(); i < hi; i += ILL_WG_THREADS) {
    const size_t r = i / per_row, c = i % per_row;
    const size_t lk = r / H.zrows, t = r % H.zrows;
    gst(a.acc + ((((size_t)other * NL) * ILL_NKIND + lk) * 16 + t) * ILL_ACC_ROW + acc_col((int)c), (uint64_t)0);
  }
}

// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void commit_apply(const IllPassArgs& a, const PassHdr& H, CommitLds& C, bool pass_kernel, int stopreq,
                                             bool kvswz = false);
// stop_word: the LDS copy of the host's stop word, loaded asynchronously by thread 0 when the
// pass started (complete once thread 0 has waited for its first poll below).
__device__ __forceinline__ void commit(const IllPassArgs& a, const PassHdr& H, CommitLds& C, const int& stop_word) {
  const uint32_t tag = tagof_lmh(H.epoch);
  const int i = tid_opaque();
  // every workgroup's partials for the rows in use (row 0 when the pass has no lm_head rows):
  // this also proves that every workgroup has read the pass header
  const int r0 = H.lmhn > 0 ? H.lmh0 : 0, nr = H.lmhn > 0 ? H.lmhn : 1;
  static_assert(ILL_WG_THREADS == 2 * ILL_WG, "thread i: workgroup i % 256, rows r0 + i / 256 + 2 m");
  // Thread i holds workgroup (i % 256)'s partials of rows r0 + (i >> 8) + 2 m (m < 8) as
  // order-preserving keys (value, lowest index), taken from the poll that saw them all, so
  // every row's partials are read in one round trip.
  uint64_t key[8];
  const bool ok = wg_wait([&]() {
    bool r = true;
#pragma unroll
    for (int m = 0; m < 8; m++) {
      const int k = i + ILL_WG_THREADS * m;
      key[m] = 0;
      if (k < ILL_WG * nr) {
        const int wgi = k % ILL_WG, t = r0 + k / ILL_WG;
        const uint64_t v = aload64(a.lmp + (wgi * 16 + t) * 2), x = aload64(a.lmp + (wgi * 16 + t) * 2 + 1);
        r &= wok(v, tag) & wok(x, tag);
        key[m] = amax_key(wval(v), (int)(uint32_t)x);
      }
    }
    return r;
  }, a.ctl, 700);
  if (!ok) return;
  trace_mark(a, ILL_TR_TAIL + 4);
  // global argmax per row: reduced in each of the 4 waves that hold a row's partials, then
  // across them
  const int lane = i & 63, wv = i >> 6;
  const int mmax = (nr + 1) >> 1;   // key[m] holds rows (i >> 8) + 2 m: only m < mmax are used
#pragma unroll
  for (int m = 0; m < 8; m++) {
    if (m >= mmax) break;   // (uniform; each 64-bit shuffle reduction is a chain of 12 ds_bpermutes)
    uint64_t k = key[m];
    for (int o = 32; o >= 1; o >>= 1) {
      const uint64_t ok2 = __shfl_xor(k, o, 64);
      k = ok2 > k ? ok2 : k;
    }
    if (lane == 0) C.key[(i >> 8) + 2 * m][wv & 3] = k;
  }
  __syncthreads();
  if (H.lmhn > 0 && i < H.lmhn) {
    uint64_t m = C.key[i][0];
    for (int ww = 1; ww < ILL_WG / 64; ww++) m = C.key[i][ww] > m ? C.key[i][ww] : m;
    C.g[H.lmh0 + i] = (int)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFu));
  }
  __syncthreads();
  commit_apply(a, H, C, true, i == 0 ? stop_word : 0);
}

// ---- drafting (k_commit_spec, Shaders.swift:367-412) ----------------------------------------
// n-gram table key of the last n tokens ctx[0..n-1], oldest first (Shaders.swift:66-70; the
// same hash as NGramTable.key, NGram.swift:13-21, so tables built by the reference load as is).
__device__ __forceinline__ uint64_t ng_key(const int* ctx, int n) {
  uint64_t h = 0xcbf29ce484222325ull ^ (uint64_t)n;
  for (int i = 0; i < n; i++) {
    h ^= (uint64_t)(uint32_t)ctx[i] + 0x9e3779b97f4a7c15ull;
    h *= 0x100000001b3ull;
    h ^= h >> 29;
  }
  return h | 1ull;
}

// Workgroup maximum of a 32-bit key (every thread gets it).
__device__ __forceinline__ uint32_t wg_max_u32(uint32_t v, uint32_t* slots) {
  const int i = threadIdx.x, w = i >> 6;
  v = group_reduce<64>(v, OpMaxU{});
  if ((i & 63) == 0) slots[w] = v;
  __syncthreads();
  uint32_t m = slots[0];
#pragma unroll
  for (int k = 1; k < ILL_WAVES; k++) m = slots[k] > m ? slots[k] : m;
  __syncthreads();
  return m;
}

// Drafts for the next pass after a speculative commit that did not stop: up to tspec - 1
// tokens (none with nodraft), each from the first source with a guess:
//   1. self-repetition: the most recent earlier occurrence of the longest suffix (3..8
//      tokens) of the recent output, continued;
//   2. the n-gram table (if one is loaded): the stored continuation of the longest known
//      context of the last 6..1 tokens (-1 before the output starts);
//   3. prompt lookup: the token after the latest longest (1..4 token) match of the output
//      suffix in the last <= 256 prompt tokens.
// Each draft is appended to the output before the next is drafted; a stop token ends the
// drafts. The reference scans with one thread, keeping the last (highest j) candidate of
// the longest match; here every thread takes one position j and the workgroup maximum of
// (match length, j) picks the same one. Then the next pass is set up as a chain over
// [last token, drafts...] with one row per token (rows, lm_head rows and commit of the
// control block, the State's n and nver).
__device__ __forceinline__ void spec_draft(const IllPassArgs& a, int have, int last, int tspec, int nodraft, int eos0, int eos1,
                                           DraftLds& D) {
  const int i = threadIdx.x;
  const int T = min(max(tspec, 1), ILL_MAXT);
  const int maxd = nodraft ? 0 : T - 1;
  if (i == 0) D.nd = 0;
  const int w0 = have > ILL_OB_MAX ? have - ILL_OB_MAX : 0;
  const int np = a.prompt && maxd > 0 ? min(max(gld(a.prompt), 0), ILL_OB_MAX) : 0;
  if (maxd > 0) {   // the window and the n-gram history (nothing to stage for a 1-row pass)
    for (int k = w0 + i; k < have; k += ILL_WG_THREADS) D.ob[k - w0] = gld(a.out_dev + k);
    if (i == 0) {
      D.L = have - w0;
      D.len = 0;
      for (int k = ILL_NG_MAXN; k >= 1; k--) D.hist[D.len++] = have - k >= 0 ? gld(a.out_dev + have - k) : -1;
    }
    __syncthreads();
  }
  for (int nd = 0; nd < maxd; nd++) {
    const int L = D.L;
    // 1. self-repetition: position j (1 <= j <= L - 1) continues a match of m >= 3 tokens
    uint32_t key = 0;
    {
      const int j = i + 1;
      if (j <= L - 1) {
        int m = 0;
        while (m < 8 && j - 1 - m >= 0 && D.ob[j - 1 - m] == D.ob[L - 1 - m]) m++;
        if (m >= 3) key = ((uint32_t)m << 16) | (uint32_t)j;
      }
    }
    key = wg_max_u32(key, D.best);
    int d = key ? D.ob[key & 0xffff] : -1;
    // 2. n-gram table: orders 6..1, 16 linear probes each, one thread per (order, probe)
    if (d < 0 && a.ngram) {
      const int len = D.len;
      if (i < ILL_NG_MAXN * 16) {
        const int n = ILL_NG_MAXN - i / 16, pr = i % 16;
        int v = 1;
        if (n <= len) {
          const uint64_t k = ng_key(D.hist + len - n, n);
          const uint32_t slot = ((uint32_t)(k >> 12) + (uint32_t)pr) & (ILL_NG_SLOTS - 1);
          const uint4 e = gld(a.ngram + slot);
          const uint64_t ek = ((uint64_t)e.y << 32) | e.x;
          v = ek == 0 ? 1 : (ek == k ? 2 + (int)e.z : 0);
        }
        D.ng[ILL_NG_MAXN - n][pr] = v;
      }
      __syncthreads();
      if (i == 0) {
        int got = -1;
        for (int n = min(ILL_NG_MAXN, len); n >= 1 && got < 0; n--)
          for (int pr = 0; pr < 16; pr++) {
            const int v = D.ng[ILL_NG_MAXN - n][pr];
            if (v == 1) break;
            if (v >= 2) { got = (unsigned)(v - 2) < (unsigned)a.W.vocab ? v - 2 : -1; break; }
          }
        D.d = got;
      }
      __syncthreads();
      d = D.d;
    }
    // 3. prompt lookup: position j (1 <= j <= np - 1) continues a match of m >= 1 tokens
    if (d < 0 && np > 1) {
      uint32_t pk = 0;
      const int j = i + 1;
      if (j <= np - 1) {
        const int32_t* P = a.prompt + 4;
        int m = 0;
        while (m < 4 && m < L && j - 1 - m >= 0 && gld(P + j - 1 - m) == D.ob[L - 1 - m]) m++;
        if (m >= 1) pk = ((uint32_t)m << 16) | (uint32_t)j;
      }
      pk = wg_max_u32(pk, D.best);
      d = pk ? gld(a.prompt + 4 + (pk & 0xffff)) : -1;
      if ((unsigned)d >= (unsigned)a.W.vocab) d = -1;   // a token outside the vocabulary is no guess
    }
    if (d < 0) break;   // uniform: every thread holds the same d
    if (i == 0) {
      D.ob[L] = d;
      D.L = L + 1;
      D.hist[D.len++] = d;
      a.ptoks[1 + nd] = d;
      D.nd = nd + 1;
    }
    __syncthreads();
    if (d == eos0 || d == eos1) break;
  }
  if (i == 0) {
    const int rows = 1 + D.nd;
    a.ptoks[0] = last;
    a.st->n = rows;
    a.st->nver = rows;
    IllCtl* c = a.ctl;
    c->mode = ILL_MODE_ROWS;
    c->nrows = rows;
    c->lmh_row0 = 0;
    c->lmh_rows = rows;
    c->commit = 2;
    c->draft = 0;
  }
}

// The drafting step after a speculative commit, as its own launch (one workgroup) so that
// the pass kernel carries none of its code: it runs when the commit left a draft pending
// (a speculative commit that did not stop) and returns at once otherwise.
__global__ __launch_bounds__(ILL_WG_THREADS) void ill_draft_kernel(IllPassArgs a) {
  __shared__ DraftLds D;
  __shared__ int go, have, last, tspec, nodraft, eos0, eos1;
  if (threadIdx.x == 0) {
    const IllState* st = a.st;
    go = a.ctl->draft && !st->done;
    have = st->step;
    last = a.ctl->last_tok;
    tspec = st->tspec;
    nodraft = st->nodraft;
    eos0 = st->eos0;
    eos1 = st->eos1;
  }
  __syncthreads();
  if (!go) return;
  spec_draft(a, have, last, tspec, nodraft, eos0, eos1, D);
}

// Cuts the drafted pass pending after a speculative commit to its first row, the last
// committed token (never a draft), so that the pass commits one token, as greedy decoding
// would, on the 1-row instantiation. A stopped request, or one whose drafting is still to
// run, is left as it is.
__global__ __launch_bounds__(64) void ill_trunc_kernel(IllPassArgs a) {
  if (threadIdx.x != 0) return;
  IllCtl* c = a.ctl;
  IllState* st = a.st;
  if (c->commit != 2 || c->draft || st->done) return;
  a.ptoks[0] = c->last_tok;
  st->n = 1;
  st->nver = 1;
  st->tree = 0;
  c->mode = ILL_MODE_ROWS;
  c->nrows = 1;
  c->lmh_row0 = 0;
  c->lmh_rows = 1;
}

// Commit of the pass's argmaxes C.g[t] (rows lmh0 ..): token record, State advance, stop
// test, chain / tree accept walk and KV compaction (Shaders.swift:192-244, :246-418). The
// pass kernel also advances the epoch and its accumulator-bank bookkeeping. The State is
// read from the header (the snapshot taken at the start of the pass: only the commit
// writes it during a pass), so the commit issues stores only.
// kvswz: the K/V cache is in the swizzled layout (q8 / f16 engines), else in rows.
__device__ __forceinline__ void commit_apply(const IllPassArgs& a, const PassHdr& H, CommitLds& C, bool pass_kernel, int stopreq,
                                             bool kvswz) {
  const int i = tid_opaque();
  IllState* st = a.st;
  if (i == 0) {
    C.npath = 0;
    C.pos0 = H.pos;
    if (stopreq) {
      // the host stopped the request (Engine.swift:1032-1036 sets the State's done flag):
      // this pass commits nothing, and every pass queued behind it leaves at its header
      st->done = 1;
      a.ctl->draft = 0;
    } else if (H.commit == 0) {
      st->pos = H.pos + H.nrows;
    } else if (H.commit == 1) {
      const int tok = C.g[H.lmh0];
      const int step = H.step;
      a.out_dev[step] = tok;
      __hip_atomic_store(a.out_host + step, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      st->step = step + 1;
      st->pos = H.pos + H.nrows;
      st->n = 1;
      // stop tokens and maxsteps (Shaders.swift:231-233); also stop before a following pass
      // of up to 16 rows would write K/V past the end of the context
      if (tok == H.eos0 || tok == H.eos1 || step + 1 >= H.maxsteps || H.pos + H.nrows + ILL_MAXT > a.maxctx) st->done = 1;
      a.ptoks[0] = tok;
      a.ctl->last_tok = tok;
    } else {
      // speculative commit (Shaders.swift:305-333): the pass's argmax rows lmh0 .. lmh0 + nv - 1
      // are [last token, drafts...]; accept the longest matching prefix (chain) or path (tree).
      // nv = 1 (a prefill, or a pass without drafts): the pass's rows are all context.
      const int nv = H.lmhn;
      const int* g = C.g + H.lmh0;
      int m = 0;
      if (H.mode == ILL_MODE_TREE) {
        int cur = 0;
        for (;;) {
          int c = -1;
          for (int r = 1; r < nv; ++r)
            if (H.parent[r] == cur && H.tok[r] == g[cur]) { c = r; break; }
          if (c < 0) break;
          C.path[m++] = c;
          cur = c;
        }
      } else {
        while (m < nv - 1 && H.tok[H.lmh0 + m + 1] == g[m]) m++;
        for (int k = 0; k < m; k++) C.path[k] = k + 1;
      }
      st->passes = H.passes + 1;
      st->accepted = H.accepted + m;
      if (a.spec_host) {   // for the host's choice of the next pass shape (Engine.swift:888-898)
        __hip_atomic_store(a.spec_host + 0, H.passes + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(a.spec_host + 1, H.accepted + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      bool stop = false;
      int last = g[0];
      int step = H.step;
      for (int k = 0; k <= m && !stop; k++) {
        const int tok = g[k == 0 ? 0 : C.path[k - 1]];
        a.out_dev[step] = tok;
        __hip_atomic_store(a.out_host + step, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        last = tok;
        if (tok == H.eos0 || tok == H.eos1 || step + 1 >= H.maxsteps) stop = true;
        step++;
      }
      const int newpos = nv == 1 ? H.pos + H.nrows : H.pos + m + 1;
      st->step = step;
      st->pos = newpos;
      st->n = 1;
      st->nver = 1;
      st->tree = 0;
      stop = stop || newpos + ILL_MAXT > a.maxctx;
      if (stop) st->done = 1;
      a.ptoks[0] = last;
      a.ctl->last_tok = last;
      C.npath = H.mode == ILL_MODE_TREE ? m : 0;
      a.ctl->draft = stop ? 0 : 1;   // ill_draft_kernel drafts the next pass
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
      kb[kv_k_off(dst, d, kvswz)] = kb[kv_k_off(src, d, kvswz)];
      uint16_t* vb = a.vt + (size_t)lh * (a.maxctx / 64) * 4096;
      vb[kv_v_off(dst, d, kvswz)] = vb[kv_v_off(src, d, kvswz)];
    }
    __syncthreads();
  }
  if (pass_kernel && i == 0) {
    a.ctl->bank_rows[H.bank] = H.nrows;   // rows of this bank to clear during the next pass
    a.ctl->bank_rows[H.bank ^ 1] = 0;     // cleared during this pass
    a.ctl->epoch = H.epoch + 1;
  }
}

// ---------------------------------------------------------------------------------------
template <int T>
__global__ __launch_bounds__(ILL_WG_THREADS, 1) void ill_pass_kernel(IllPassArgs args) {
  // A private copy: the roles take the arguments by reference, and a reference to the
  // kernel-argument segment would otherwise be re-read with FLAT loads inside hot loops.
  const IllPassArgs a = args;
  __shared__ PassLds<T> S;
  extern __shared__ __attribute__((aligned(16))) uint8_t ill_stage[];   // ILL_STAGE_BYTES (dynamic)
  __shared__ PassHdr H;
  trace_mark(a, ILL_TR_TAIL + 8);
  // the kernel arguments the header and the first weight stage use, read in one batch of
  // scalar loads before the header (left to the compiler, they came in several dependent
  // rounds: 1 us per step; adding the arguments the roles use next measured slower)
  asm volatile("" ::"s"(a.st), "s"(a.ctl), "s"(a.ptoks), "s"(a.tree), "s"(a.L0.wqkv), "s"(a.L0.sqkv), "s"(a.L0.wo),
               "s"(a.L0.so), "s"(a.L0.wgu), "s"(a.L0.sgu), "s"(a.L0.wd), "s"(a.L0.sd));
  load_hdr(a, H);
  trace_mark(a, ILL_TR_TAIL + 9);
  if (H.done) return;
  // The host's stop word, for the commit (workgroup 0): copied into LDS by an asynchronous
  // load issued now and used at the end of the pass, so its round trip to host memory stays
  // off the critical path and no register holds it meanwhile.
  __shared__ int stop_lds;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    if (a.stop_host)
      __builtin_amdgcn_global_load_lds((const void*)a.stop_host, (__attribute__((address_space(3))) void*)&stop_lds, 4, 0,
                                       ILL_BUF_SYS);
    else
      stop_lds = 0;
  }
  // a pass must fit this instantiation: every workgroup reads the same header and leaves
  if (H.nrows < 1 || H.nrows > T || H.lmhn < 0 || H.lmh0 < 0 || H.lmh0 + H.lmhn > T) {
    if (blockIdx.x == 0 && threadIdx.x == 0) set_err(a.ctl, ILL_ERR_SHAPE);
    return;
  }
  const int wg = blockIdx.x;
  const int NL = a.W.layers;
  const int tid = tid_opaque(), w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool att0 = wg >= ILL_R_ATT0 && wg < ILL_R_ATT0 + ILL_NATT;
  const bool att1 = ill_pub<T>() && wg >= ILL_R_ATT1 && wg < ILL_R_ATT1 + ILL_NATT;
  if (att0 || att1) {
    const int h = att0 ? wg - ILL_R_ATT0 : wg - ILL_R_ATT1, half = att0 ? 0 : 1;
    att_stage_qkv<T>(a.L0, h, w, lane, ill_stage);
    if (T == 1) att_stage_o<T>(a.L0, h, w, lane, ill_stage);
    for (int l = 0; l < NL; l++) {
      trace_mark(a, ILL_TRL * l);
      if (!role_att<T>(a, H, S.att, l, h, half, ill_stage)) return;
      lds_barrier();   // every wave is done with the stage before it is refilled
      if (l + 1 < NL) {
        const IllLayerW Ln = layer_ptrs(a.L, l + 1);
        const IllLayerW& L1 = T == 1 ? a.L[l + 1] : Ln;
        att_stage_qkv<T>(L1, h, w, lane, ill_stage);
        if (T == 1) att_stage_o<T>(L1, h, w, lane, ill_stage);
      }
      trace_mark(a, ILL_TRL * l + 11);
    }
  } else if (wg >= ILL_R_GUD0 && wg < ILL_R_GUD0 + ILL_NGU) {
    const int ub = wg - ILL_R_GUD0;
    gud_stage(a.L0, ub, w, lane, ill_stage);
    for (int l = 0; l < NL; l++) {
      trace_mark(a, ILL_TRL * l);
      if (!role_gud<T>(a, H, S.gud, l, ub, ill_stage)) return;
      lds_barrier();
      if (l + 1 < NL) {
        const IllLayerW Ln = layer_ptrs(a.L, l + 1);
        gud_stage(T == 1 ? a.L[l + 1] : Ln, ub, w, lane, ill_stage);
      }
      trace_mark(a, ILL_TRL * l + 11);
    }
  } else if (!ill_pub<T>() && wg == ILL_R_BASE) {   // (16-row passes: REDUCE keeps the residual)
    for (int l = 0; l < NL; l++) {
      trace_mark(a, ILL_TRL * l);
      if (!role_base<T>(a, H, l)) return;
      trace_mark(a, ILL_TRL * l + 11);
    }
  } else if (ill_pub<T>() && wg >= ILL_R_RED0 && wg < ILL_R_RED0 + ILL_NRED) {
    if (!role_red<T>(a, H, wg - ILL_R_RED0, ill_stage)) return;
  } else if (ill_pub<T>() && wg >= ILL_R_PREP0 && wg < ILL_R_PREP0 + ILL_MAXT) {
    const int t = wg - ILL_R_PREP0;
    if (t < H.nrows) {
      if (!role_prep<T>(a, H, S.prep1, t)) return;
      lds_barrier();
    }
  }
  trace_mark(a, ILL_TR_TAIL);
  if (!role_lmh<T>(a, H, S.lmh, ill_stage)) return;
  if (wg != 0) zero_other_bank(a, H);
  trace_mark(a, ILL_TR_TAIL + 2);
  if (wg == 0) {   // the commit first: the bank is next used by the following launch
    __syncthreads();
    commit(a, H, S.cm, stop_lds);
    trace_mark(a, ILL_TR_TAIL + 5);
    zero_other_bank(a, H);
  }
  trace_mark(a, ILL_TR_TAIL + 10);
}
