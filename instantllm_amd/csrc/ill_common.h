// Shared host/device definitions of the MI355X decode engine.
//
// Model shape is fixed like the reference engine (Sources/Engine/Shaders.swift:12-21):
// hidden 896, FFN 4864, 14 query heads, 2 KV heads, head_dim 64, QKV rows 1152. The layer
// count and vocabulary come from the .ill file (24 / 151936 for the real model).
#pragma once
#include <stdint.h>

#define ILL_H 896
#define ILL_FF 4864
#define ILL_NH 14
#define ILL_NKV 2
#define ILL_HD 64
#define ILL_QKV 1152
#define ILL_EPS 1e-6f
#define ILL_MAXT 16          // rows per pass (1-row decode .. 16-row tree verify)
#define ILL_MAXLAYERS 30

// Device layout unit sizes (q4): a "block" is 16 rows x 128 columns = 2 quant groups.
#define ILL_KST 7            // 896 / 128 column blocks per K = 896 row tile
#define ILL_NGU 76           // 4864 / 64 hidden-unit blocks of the fused gate/up/down role
// The residual accumulators of a 1-row pass are kept in copies that their readers add up:
// fewer contributors per cache line, so the atomics land sooner. The post-attention
// residual XA has ILL_XA_COPIES (head h adds into copy h % ILL_XA_COPIES), the post-MLP
// residual XB ILL_XB_COPIES (unit block ub into copy ub % ILL_XB_COPIES); the base adds
// into copy 0 of each.
#ifndef ILL_XA_COPIES
#define ILL_XA_COPIES 2
#endif
#ifndef ILL_XB_COPIES
#define ILL_XB_COPIES 2
#endif
#define ILL_NKIND (ILL_XA_COPIES + ILL_XB_COPIES)   // accumulator kinds per layer: XA, XB copies
#define ILL_NOT 56           // 896 / 16 row tiles of O and down
#define ILL_NQB 36           // 1152 / 32 rotary blocks of QKV

// Persistent-kernel geometry (WG i runs on XCD i % 8, so consecutive WG ranges are
// spread over all eight XCDs).
#define ILL_WG 256           // workgroups (one per CU on MI355X)
#define ILL_WG_THREADS 512   // 8 waves
#define ILL_WAVES 8

// K/V cache: per (layer, KV head), blocks of 64 slots of 4096 halves. Offsets in halves
// from the (layer, head) base, in two layouts:
//  - rows (the q4 engine, whose pass kernel reads 16 keys x 64 dims fragments for MFMA):
//      K (slot s, dim d): s * 64 + d;  V (slot s, dim d): (s >> 6) * 4096 + d * 64 + (s & 63)
//  - swizzled (q8 and f16, whose attention kernels give each lane one key or one dim):
//    K dim-group major and V position-group major inside a block, so that 64 lanes reading
//    16 bytes each for 64 consecutive slots (K: one key per lane, 8 dims) or 64 dims (V: one
//    dim per lane, 8 positions) read 1 KB contiguous:
//      K: (s >> 6) * 4096 + ((d >> 3) * 64 + (s & 63)) * 8 + (d & 7)
//      V: (s >> 6) * 4096 + (((s & 63) >> 3) * 64 + d) * 8 + (s & 7)
__host__ __device__ inline size_t kv_k_off(int s, int d, bool swz) {
  return swz ? (size_t)(s >> 6) * 4096 + (size_t)((((d >> 3) << 6) + (s & 63)) << 3) + (d & 7) : (size_t)s * 64 + d;
}
__host__ __device__ inline size_t kv_v_off(int s, int d, bool swz) {
  return swz ? (size_t)(s >> 6) * 4096 + (size_t)((((s & 63) >> 3 << 6) + d) << 3) + (s & 7)
             : (size_t)(s >> 6) * 4096 + d * 64 + (s & 63);
}

// State: the reference's 16-int control block (Shaders.swift:37-54), same field order.
struct IllState {
  int32_t pos, n, step, done, maxctx, maxsteps, eos0, eos1;
  int32_t nver, tspec, passes, accepted, tlmh, nodraft, learned, tree;
};

// Engine-private control block (device memory).
struct IllCtl {
  uint32_t epoch;       // pass counter; tags are epoch * 32 + layer + 1
  int32_t err;          // nonzero: a bounded wait timed out (code = where)
  int32_t mode;         // pass mode of the kernel in flight
  int32_t nrows;        // valid rows of the pass
  int32_t lmh_row0;     // first row whose logits/argmax the pass computes
  int32_t lmh_rows;     // rows of the lm_head
  int32_t write_logits;
  int32_t commit;       // 0: advance pos only (prefill chunk), 1: greedy commit, 2: spec commit
  int32_t last_tok;     // last committed token (decode input)
  int32_t bank_rows[2]; // rows of each residual-accumulator bank still to be cleared
  int32_t draft;        // a speculative commit left the next pass's drafting to a drafting kernel
  int32_t tree_b;       // learned drafter: > 0 drafts a best-first tree of this many tokens
  int32_t pad[3];
};

enum IllMode { ILL_MODE_DECODE = 0, ILL_MODE_ROWS = 1, ILL_MODE_TREE = 2 };

// Tree buffer layout (Shaders.swift:23-30): [n, depth[16], parent[16], tok[16], anc[16]].
#define ILL_TR_DEPTH 1
#define ILL_TR_PARENT 17
#define ILL_TR_TOK 33
#define ILL_TR_ANC 49
#define ILL_TR_INTS 65

// Per-layer device weight pointers (repacked layout).
struct IllLayerW {
  const uint8_t* wqkv;   const uint32_t* sqkv;   // 72 row tiles x 7 blocks
  const uint8_t* wo;     const uint32_t* so;     // 14 column groups (heads) x 56 row tiles (512 B each)
  const uint8_t* wgu;    const uint32_t* sgu;    // 76 unit blocks x 8 tiles x 7 blocks
  const uint8_t* wd;     const uint32_t* sd;     // 76 column groups x 56 row tiles (512 B each)
  const float* bqkv;     // 1152, stored (rotary block) order
  const float* ln1;
  const float* ln2;
};

struct IllWeights {
  const uint8_t* wemb; const uint32_t* semb;   // V/16 row tiles x 7 blocks (tied lm_head)
  const float* fnorm;
  int32_t vocab;
  int32_t layers;
  int32_t fmt;
};
