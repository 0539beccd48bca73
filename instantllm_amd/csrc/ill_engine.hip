// Host engine of the MI355X decode path and the C ABI of include/ill_hip.h.
//
// Mirrors the reference's Swift Engine (Sources/Engine/Engine.swift): it maps the .ill
// file, owns the device buffers and the device State, and encodes passes. Each pass is a
// single persistent kernel launch (ill_pass.h); decode steps are recorded into hipGraphs
// so the generate loop never returns to the host between tokens.
#include <hip/hip_runtime.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ill_hip.h"
#include "ill_pass.h"
#include "ill_gemv.h"
#include "ill_ops.h"
#include "ill_quant.h"
#include "ill_ildraft_host.h"
#include "ill_tok.h"

namespace {

thread_local std::string g_err = "no error";

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HCK(x)                                                                            \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) return fail(ILL_E_HIP, "%s: %s (%s:%d)", #x, hipGetErrorString(e_), __FILE__, __LINE__); \
  } while (0)

constexpr uint32_t kMagic = 0x314D4C49;   // "ILM1" (ModelFile.swift:62)
constexpr int kHeader = 16384;

struct Mapped {
  void* base = nullptr;
  size_t len = 0;
  ~Mapped() {
    if (base) munmap(base, len);
  }
};

// ---- repacking of the .ill tensors into the device tile layout ------------------------
// q4 row tile: block (rt, cb) = 1 KiB; lane l = 16 kg + n stores 8 bytes of row n at
// columns 128 cb + 16 kg (group 2 cb) then 8 bytes at 128 cb + 64 + 16 kg (group 2 cb + 1).
void repack_rows(const uint8_t* w, const uint32_t* sb, int K, const std::vector<int>& rows, uint8_t* dw, uint32_t* ds) {
  const int nb = K / 128, rb = K / 2, sg = K / 64;
  const int ntile = (int)rows.size() / 16;
  for (int rt = 0; rt < ntile; rt++)
    for (int cb = 0; cb < nb; cb++) {
      uint8_t* blk = dw + ((size_t)rt * nb + cb) * 1024;
      uint32_t* sblk = ds + ((size_t)rt * nb + cb) * 32;
      for (int l = 0; l < 64; l++) {
        const int kg = l >> 4, n = l & 15;
        const int r = rows[16 * rt + n];
        memcpy(blk + l * 16, w + (size_t)r * rb + (128 * cb + 16 * kg) / 2, 8);
        memcpy(blk + l * 16 + 8, w + (size_t)r * rb + (128 * cb + 64 + 16 * kg) / 2, 8);
      }
      for (int n = 0; n < 16; n++) {
        const int r = rows[16 * rt + n];
        sblk[n * 2 + 0] = sb[(size_t)r * sg + 2 * cb];
        sblk[n * 2 + 1] = sb[(size_t)r * sg + 2 * cb + 1];
      }
    }
}

// Split-K layout of a [896][K] projection (O: K = 896, down: K = 4864): block (G, rt) =
// 512 B; lane l = 16 kg + n stores 8 bytes of row 16 rt + n at columns 64 G + 16 kg;
// scales [G][rt][n]. A workgroup owning column group G reads one contiguous 28 KiB run.
void repack_split(const uint8_t* w, const uint32_t* sb, int K, uint8_t* dw, uint32_t* ds) {
  const int rb = K / 2, sg = K / 64;
  for (int G = 0; G < sg; G++)
    for (int rt = 0; rt < ILL_NOT; rt++) {
      uint8_t* blk = dw + ((size_t)G * ILL_NOT + rt) * 512;
      for (int l = 0; l < 64; l++) {
        const int kg = l >> 4, n = l & 15;
        memcpy(blk + l * 8, w + (size_t)(16 * rt + n) * rb + (64 * G + 16 * kg) / 2, 8);
      }
      for (int n = 0; n < 16; n++) ds[((size_t)G * ILL_NOT + rt) * 16 + n] = sb[(size_t)(16 * rt + n) * sg + G];
    }
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

struct ill_engine {
  int fmt = 2, layers = 0, vocab = 0, maxctx = 0, maxpass = 16, maxsteps = 0;
  std::string path;   // the model file (the prefix-cache key)
  hipStream_t stream = nullptr;
  uint8_t* dweights = nullptr;
  IllLayerW* dlayers = nullptr;
  IllWeights W{};
  std::vector<IllLayerW> hlayers;
  IllState* st = nullptr;
  IllCtl* ctl = nullptr;
  int32_t* ptoks = nullptr;
  int32_t* tree = nullptr;
  float2* rope = nullptr;
  uint16_t* kc = nullptr;
  uint16_t* vt = nullptr;
  uint64_t *acc = nullptr, *lmp = nullptr, *pub = nullptr;
  uint4* part = nullptr;   // 16-row passes: down-projection partials (ILL_PART_WORDS 16-byte words)
  size_t acc_bytes = 0;
  float* logits = nullptr;
  int32_t* out_dev = nullptr;
  int32_t* out_host = nullptr;
  int32_t* spec_host = nullptr;   // pinned [2]: passes, accepted drafts (written by spec commits)
  int32_t* stop_host = nullptr;   // pinned, host-coherent: the stop request read by each commit
  int32_t* prompt = nullptr;      // [4 + 256]: prompt-lookup context of the drafter
  uint8_t* ngram = nullptr;       // n-gram draft table (ILL_NG_SLOTS x 16 B), optional
  // learned drafter (ILDraft.swift): host table, device copies, per-request context
  illd::Table* ild = nullptr;
  uint8_t* dtab = nullptr;
  uint8_t* dtflg = nullptr;
  IllDraftReq* dreq = nullptr;
  IllDraftArgs dargs{};
  bool draft_ctx_ready = false;   // a context was prepared for the next generate_spec call
  bool learned_active = false;    // the State's `learned`: commits leave drafting to ill_ildraft_kernel
  bool use_learned = true;
  int learned_T = 8, learned_tree = 15;
  bool graph_spec = false;        // the captured graph holds spec passes (their control comes from the device)
  int graph_T = 0;                // pass instantiation of the captured spec graph
  bool graph_learned = false;     // its drafting kernel is the learned drafter's
  // generate_spec's own graphs of chained passes, one per pass instantiation (1, 4, 16 rows)
  struct SpecGraph {
    hipGraph_t g = nullptr;
    hipGraphExec_t x = nullptr;
    int steps = 0;
    bool learned = false;
  } sg[3];
  // Engine.cachedTokens (Engine.swift:929-933, :1029-1031): tokens whose K/V are valid at
  // positions 0.. after the last generate call; any pass launched outside generate clears it
  std::vector<int32_t> cached;
  bool in_generate = false;
  int last_prefill = 0;           // tokens the last generate call prefilled
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  int graph_steps = 0;
  uint64_t passes_since_clear = 0;   // passes launched since the tagged buffers were cleared
  int pos_hint = 0;   // the State's pos as the host last knew it: picks the attention split
  IllCtl hctl{};
  IllPassArgs args{};
  int logits_rows_valid = 0;
  // layer-by-layer path (prefill chunks > 16 rows; every pass of q8 / f16 models)
  uint8_t* oweights = nullptr;
  OpLayerW* dolayers = nullptr;
  std::vector<OpLayerW> holayers;
  OpCtx octx{};
  float* opart = nullptr;   // split-K partials of the layer-by-layer GEMMs
  int q8g = 64;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;   // bracket the last single-pass launch
};

namespace {

// A pass or cache write from outside generate: the generate prefix cache no longer holds.
void touch_cache(ill_engine* e) {
  if (!e->in_generate) e->cached.clear();
}

int set_ctl(ill_engine* e, int mode, int nrows, int lmh0, int lmhn, int wlog, int commit) {
  IllCtl c{};
  c.mode = mode;
  c.nrows = nrows;
  c.lmh_row0 = lmh0;
  c.lmh_rows = lmhn;
  c.write_logits = wlog;
  c.commit = commit;
  // epoch / err / last_tok are device-owned: write only the host fields (offset 8..)
  e->hctl = c;
  HCK(hipMemcpyAsync((char*)e->ctl + offsetof(IllCtl, mode), (char*)&e->hctl + offsetof(IllCtl, mode),
                     offsetof(IllCtl, last_tok) - offsetof(IllCtl, mode), hipMemcpyHostToDevice, e->stream));
  return 0;
}

int count_passes(ill_engine* e, int n);

// The pass-kernel instantiation for a pass of `rows` rows: 1, up to 4, up to 16 (a row's
// arithmetic is the same in each).
// The smallest instantiation for a pass of `rows` rows, except that 3- and 4-row passes take
// the 16-row kernel: with its publications and reducers it measured faster for them (763
// against 804 us at 4 rows, 742 against 759 at 3; 722 against 710 at 2).
int pass_T(int rows) { return rows <= 1 ? 1 : (rows <= 2 ? 4 : 16); }

void op_seq_fmt(ill_engine* e, int M, int lm_rows);

// One pass of up to T rows whose rows, mode and commit come from the device (the control
// block the previous commit or the host wrote): q4 on the T-row pass kernel; q8 and f16 on
// the layer-by-layer kernels launched for T rows, of which the rows beyond the pass's own
// are computed and never committed (row t's K/V slot is pos + t, so they touch no live
// slot, and every row's arithmetic is independent of the others).
void enqueue_pass(ill_engine* e, int T) {
  if (e->fmt != 2) op_seq_fmt(e, T, T);
  else if (T == 1) hipLaunchKernelGGL(ill_pass_kernel<1>, dim3(ILL_WG), dim3(ILL_WG_THREADS), ill_stage_bytes(1), e->stream, e->args);
  else if (T == 4) hipLaunchKernelGGL(ill_pass_kernel<4>, dim3(ILL_WG), dim3(ILL_WG_THREADS), ill_stage_bytes(4), e->stream, e->args);
  else hipLaunchKernelGGL(ill_pass_kernel<16>, dim3(ILL_WG), dim3(ILL_WG_THREADS), ill_stage_bytes(16), e->stream, e->args);
}

int launch(ill_engine* e, int T) {
  if (int rc = count_passes(e, 1)) return rc;
  HCK(hipEventRecord(e->ev0, e->stream));
  enqueue_pass(e, T);
  HCK(hipGetLastError());
  HCK(hipEventRecord(e->ev1, e->stream));
  return 0;
}

// The drafting kernel after a launch whose commit is speculative (it returns at once unless
// that commit left a draft pending): the learned drafter's while the State says so, else the
// commit's own drafting (self-repetition, n-gram table, prompt lookup).
void enqueue_draft(ill_engine* e) {
  if (e->learned_active)
    hipLaunchKernelGGL(ill_ildraft_kernel, dim3(1), dim3(ILD_THREADS), 0, e->stream, e->args, e->dargs);
  else
    hipLaunchKernelGGL(ill_draft_kernel, dim3(1), dim3(ILL_WG_THREADS), 0, e->stream, e->args);
}

int launch_draft(ill_engine* e) {
  enqueue_draft(e);
  HCK(hipGetLastError());
  return 0;
}

int check_err(ill_engine* e) {
  int32_t err = 0;
  HCK(hipMemcpyAsync(&err, &e->ctl->err, 4, hipMemcpyDeviceToHost, e->stream));
  HCK(hipStreamSynchronize(e->stream));
  if (err) {
    // An abandoned pass leaves partial sums behind (clear both accumulator banks) and tagged
    // words of its own epoch in the published codings, the down-projection partials and the
    // lm_head partials: the epoch
    // moves on by two (the same bank parity), so the next pass's tags differ from them.
    uint32_t ep = 0;
    hipMemcpy(&ep, &e->ctl->epoch, 4, hipMemcpyDeviceToHost);
    ep += 2;
    int32_t zero[3] = {0, 0, 0};
    hipMemcpy(&e->ctl->epoch, &ep, 4, hipMemcpyHostToDevice);
    hipMemcpy(&e->ctl->err, zero, 4, hipMemcpyHostToDevice);
    hipMemcpy(&e->ctl->bank_rows[0], zero, 8, hipMemcpyHostToDevice);
    hipMemset(e->acc, 0, e->acc_bytes);
    hipDeviceSynchronize();
    if (err == ILL_ERR_SHAPE) return fail(ILL_E_ARG, "a pass had more rows than its kernel instantiation; it was abandoned");
    return fail(ILL_E_TIMEOUT, "device wait timed out (site %d); the pass was abandoned", err);
  }
  return 0;
}

// Tags are 32-bit (epoch * 32 + slot + 1), so they repeat every 2^27 passes. Words that
// are not rewritten for that long (rows 1-15 of the published codings, written by 16-row
// passes only) could then pass a tag check: the host clears both tagged buffers once
// every ILL_TAG_CLEAR_PASSES launched passes, long before a tag can come round again.
#define ILL_TAG_CLEAR_PASSES (1u << 24)
int count_passes(ill_engine* e, int n) {
  e->passes_since_clear += (uint64_t)n;
  if (e->passes_since_clear < ILL_TAG_CLEAR_PASSES) return 0;
  HCK(hipStreamSynchronize(e->stream));
  HCK(hipMemsetAsync(e->pub, 0, (size_t)ILL_PUB_WORDS * 8, e->stream));
  HCK(hipMemsetAsync(e->part, 0, (size_t)ILL_PART_WORDS * 16, e->stream));
  HCK(hipMemsetAsync(e->lmp, 0, (size_t)ILL_WG * 16 * 2 * 8, e->stream));
  HCK(hipStreamSynchronize(e->stream));
  e->passes_since_clear = (uint64_t)n;
  return 0;
}

void drop_graph(ill_engine* e) {
  if (e->gexec) hipGraphExecDestroy(e->gexec);
  if (e->graph) hipGraphDestroy(e->graph);
  e->gexec = nullptr;
  e->graph = nullptr;
  e->graph_steps = 0;
  e->graph_T = 0;
  for (auto& g : e->sg) {
    if (g.x) hipGraphExecDestroy(g.x);
    if (g.g) hipGraphDestroy(g.g);
    g = ill_engine::SpecGraph{};
  }
}

int read_state(ill_engine* e, IllState* s) {
  HCK(hipMemcpyAsync(s, e->st, sizeof(IllState), hipMemcpyDeviceToHost, e->stream));
  HCK(hipStreamSynchronize(e->stream));
  return 0;
}

int write_pos_n(ill_engine* e, int pos, int n) {
  int32_t v[2] = {pos, n};
  HCK(hipMemcpyAsync(e->st, v, 8, hipMemcpyHostToDevice, e->stream));
  return 0;
}

// ---- layer-by-layer path -----------------------------------------------------------------
// Passes of up to 16 rows: the GEMMs that are not register-direct GEMVs (the lm_head, and the
// gate/up GEMM with K split) run on the LDS-ring GEMM for q8 and f16, on op_gemm_kernel for
// q4. q8 dequantizes its weights as they leave the ring instead of into an LDS tile: q8
// decode after 512 positions 892 -> 859 us, at 4096 1,004 -> 975 us (the lm_head alone
// 4 us of it). f16 takes a ring of 4 stages here (with the prefill gate/up's 2 it was 14 us
// slower than op_gemm_kernel; with 4, 873 -> 855 us, at 4096 991 -> 973 us).
#define OP_SMALL_RING(FMT) ((FMT) != 2)
#ifndef OP_RING_ST_SMALL_F16
#define OP_RING_ST_SMALL_F16 4
#endif
#define OP_RING_ST_SMALL(FMT, EPI) ((FMT) == 0 ? OP_RING_ST_SMALL_F16 : OP_RING_ST(FMT, EPI))
#define ILL_OP_PART_BYTES (16u << 20)   // >= slices x rows x N x 4 of every split GEMM
#define ILL_OP_PART_SPLIT (2u << 20)    // floats: passes of up to 16 rows keep the gate/up
                                        // partials below, the down GEMM's above

// Returns true when it also wrote the RMSNorm of the updated residual (rows >= norm_row0,
// weights norm_gamma) into xn: residual GEMMs of passes of up to 16 rows with K split.
// Passes of up to 16 rows only: a gate/up GEMM given silu_out leaves its K-slice partials
// in opart for the down GEMM and stores their count there (0: it applied SiLU itself); a
// residual GEMM given silu_S > 0 takes its A operand from those partials.
template <int FMT, int EPI>
bool op_gemm(ill_engine* e, const __half* A, const OpMat& W, int M, int layer, float* resid,
             const float* norm_gamma = nullptr, int norm_row0 = 0, int* silu_out = nullptr, int silu_S = 0) {
  OpGemmArgs g;
  g.c = e->octx;
  g.A = A;
  g.W = W;
  g.M = M;
  g.layer = layer;
  g.resid = resid;
  g.part = e->opart;
  g.pos_hint = e->pos_hint;
  const int nsteps = W.K / OP_BK, ntn = W.N / OP_BN;
  if constexpr (EPI != OP_LMH) {
    if (M > 16) {   // prefill chunk: 64-row tiles, K split only where the tiles are few
      if (EPI == OP_QKV) {
        // QKV: 16-row tiles over the whole K and the epilogue in the GEMM (no partials and no
        // reduction kernel): 512 rows, f16, 13.9 us against 9.7 + 5.4 us split three ways
        g.ksteps = nsteps;
        if constexpr (FMT != 2)   // q8 / f16: 32-row tiles streamed through the LDS ring
          hipLaunchKernelGGL((op_gemm_ring_kernel<FMT, 32, EPI, OP_RING_ST(FMT, EPI)>), dim3(ntn, (M + 31) / 32, 1), dim3(256), 0,
                             e->stream, g);
        else
          hipLaunchKernelGGL((op_gemm_kernel<FMT, 16, EPI, 4>), dim3(ntn, (M + 15) / 16, 1), dim3(256), 0, e->stream, g);
        return false;
      }
      const int mt = (M + 63) / 64;
      const int cap = (int)(ILL_OP_PART_BYTES / ((size_t)M * W.N * 4));   // partial buffer
      int S = std::max(1, std::min(std::min(std::min(256 / (ntn * mt), nsteps / 4), OP_MAXS), cap));
      g.ksteps = (nsteps + S - 1) / S;
      S = (nsteps + g.ksteps - 1) / g.ksteps;
      // the many-tile gate/up GEMM streams best with the one-step kernel (more per CU)
      if constexpr (FMT != 2)
        hipLaunchKernelGGL((op_gemm_ring_kernel<FMT, 64, EPI, OP_RING_ST(FMT, EPI)>), dim3(ntn, mt, S), dim3(256), 0, e->stream, g);
      else
        hipLaunchKernelGGL((op_gemm_kernel<FMT, 64, EPI, EPI == OP_SILU ? 1 : 4>), dim3(ntn, mt, S), dim3(256), 0, e->stream, g);
      if (S > 1) {
        if (EPI == OP_RESID && norm_gamma && W.N == ILL_H) {
          hipLaunchKernelGGL(op_epi_norm_kernel, dim3(M), dim3(ILL_H), 0, e->stream, g, S, norm_gamma, norm_row0);
          return true;
        }
        const int per = EPI == OP_RESID ? W.N : W.N / 2;
        hipLaunchKernelGGL((op_epi_kernel<EPI>), dim3((M * per + 255) / 256), dim3(256), 0, e->stream, g, S);
      }
      return false;
    }
  }
  // up to 16 rows: split K so that about 256 workgroups stream the weights,
  // at least four k-steps per slice (the split depends on the matrix only, so 1-row and
  // 16-row passes sum the same partials in the same order)
  int S = 1;
  // (QKV of q8 / f16: K not split across workgroups; 36 two-wave workgroups, each wave half
  // of K, apply the epilogue themselves)
  constexpr bool QKV1 = EPI == OP_QKV && FMT != 2;
  if (EPI != OP_LMH && !QKV1) S = std::max(1, std::min(std::min((256 + ntn - 1) / ntn, nsteps / 4), OP_MAXS));
  g.ksteps = (nsteps + S - 1) / S;
  S = (nsteps + g.ksteps - 1) / g.ksteps;
  if (g.ksteps * OP_BK > OP_SMAXK) {
    fail(ILL_E_ARG, "K slice of %d columns exceeds %d", g.ksteps * OP_BK, OP_SMAXK);
    return false;
  }
  const dim3 grid(ntn, 1, S);
  if (EPI == OP_RESID && silu_S > 0) {   // A = SwiGLU of the gate/up partials left in opart
    g.apart = e->opart;
    g.aS = silu_S;
    g.part = e->opart + ILL_OP_PART_SPLIT;
    hipLaunchKernelGGL((op_gemv_kernel<FMT, EPI, true>), grid, dim3(256), 0, e->stream, g);
  } else if constexpr (QKV1) {
    hipLaunchKernelGGL((op_gemv_kernel<FMT, EPI, false, 2>), dim3(W.N / 32), dim3(128), 0, e->stream, g);
  } else if constexpr (OP_SMALL_RING(FMT)) {
    hipLaunchKernelGGL((op_gemm_ring_kernel<FMT, 16, EPI, OP_RING_ST_SMALL(FMT, EPI)>), grid, dim3(256), 0, e->stream, g);
  } else {
    hipLaunchKernelGGL((op_gemm_kernel<FMT, 16, EPI, 4>), grid, dim3(256), 0, e->stream, g);
  }
  if constexpr (EPI != OP_LMH) {
    if (S > 1) {
      if (EPI == OP_SILU && silu_out && (size_t)S * M * W.N * 4 <= ILL_OP_PART_SPLIT * 4) {
        *silu_out = S;   // the down GEMM takes the partials
        return false;
      }
      if (EPI == OP_RESID && norm_gamma && W.N == ILL_H) {
        hipLaunchKernelGGL(op_epi_norm_kernel, dim3(M), dim3(ILL_H), 0, e->stream, g, S, norm_gamma, norm_row0);
        return true;
      }
      const int per = EPI == OP_RESID ? W.N : W.N / 2;
      hipLaunchKernelGGL((op_epi_kernel<EPI>), dim3((M * per + 255) / 256), dim3(256), 0, e->stream, g, S);
    }
  }
  return false;
}

// The kernels of one pass over M rows (control block and State already written): layers,
// lm_head on the last lm_rows rows (0: none), commit.
template <int FMT>
void op_seq(ill_engine* e, int M, int lm_rows) {
  const OpCtx& c = e->octx;
  hipStream_t s = e->stream;
  // the embedding with layer 0's RMSNorm (one launch)
  hipLaunchKernelGGL(op_embed_norm_kernel<FMT>, dim3((M + 3) / 4), dim3(256), 0, s, c, e->holayers[0].ln1, M);
  // passes of up to 16 rows: attention split over up to 8 workgroups per (row, head), one
  // per 1024 positions of context (the result does not depend on the split)
  const int nch = (e->pos_hint + M + 63) / 64;
  const int nsplit = std::max(1, std::min(OP_NSPLIT, (nch + 15) / 16));
  // passes of up to 16 rows (q8 / f16; q4 ones run on the pass kernel): the O projection
  // runs per head inside the attention kernel (one split) or the split combine, always with
  // the same arithmetic, so the split does not change the result
  const bool ofuse = FMT != 2 && M <= 16;
  float* opart_o = e->opart + ILL_OP_PART_SPLIT;   // [head][row][896] O partials
  // each residual update also writes the next RMSNorm where its K is split (op_gemm returns
  // whether it did)
  bool normed = true;   // (layer 0's came with the embedding)
  for (int l = 0; l < e->layers; l++) {
    const OpLayerW& L = e->holayers[l];
    if (!normed) hipLaunchKernelGGL(op_norm_kernel, dim3((M + 3) / 4), dim3(256), 0, s, c, L.ln1, 0, M);
    op_gemm<FMT, OP_QKV>(e, c.xn, L.qkv, M, l, nullptr);
    if (M > 16) hipLaunchKernelGGL(op_attn_rows_kernel<FMT != 2>, dim3((M + 15) / 16, ILL_NH), dim3(64 * OP_RW), 0, s, c, l, M);
    else {
      float* op1 = ofuse && nsplit == 1 ? opart_o : nullptr;
      hipLaunchKernelGGL(op_attn_kernel<FMT>, dim3(M * ILL_NH * nsplit), dim3(64 * ILL_WAVES), 0, s, c, l, M, nsplit, e->opart,
                         L.oh, op1);
      if (nsplit > 1)
        hipLaunchKernelGGL(op_attn_combine_kernel<FMT>, dim3(M * ILL_NH), dim3(64 * ILL_WAVES), 0, s, c, (const float*)e->opart,
                           L.oh, ofuse ? opart_o : (float*)nullptr, M);
      if (ofuse) {   // the residual + norm over the 14 per-head O partials (head order)
        OpGemmArgs g{};
        g.c = c;
        g.W = L.o;
        g.M = M;
        g.layer = l;
        g.resid = c.x;
        g.part = opart_o;
        hipLaunchKernelGGL(op_epi_norm_kernel, dim3(M), dim3(ILL_H), 0, s, g, ILL_NH, L.ln2, 0);
      }
    }
    const bool fuse = M <= 16;   // the SwiGLU hand-over (the residual + norm fusion: any M)
    if (!ofuse && !op_gemm<FMT, OP_RESID>(e, c.ao, L.o, M, l, c.x, L.ln2, 0))
      hipLaunchKernelGGL(op_norm_kernel, dim3((M + 3) / 4), dim3(256), 0, s, c, L.ln2, 0, M);
    int silu_S = 0;
    op_gemm<FMT, OP_SILU>(e, c.xn, L.gu, M, l, nullptr, nullptr, 0, fuse ? &silu_S : nullptr);
    const bool last = l + 1 == e->layers;
    const float* next = last ? (lm_rows > 0 ? c.fnorm : nullptr) : e->holayers[l + 1].ln1;
    normed = op_gemm<FMT, OP_RESID>(e, c.h, L.d, M, l, c.x, next, last ? M - lm_rows : 0, nullptr, silu_S);
  }
  if (lm_rows > 0) {
    if (!normed) hipLaunchKernelGGL(op_norm_kernel, dim3((lm_rows + 3) / 4), dim3(256), 0, s, c, c.fnorm, M - lm_rows, lm_rows);
    op_gemm<FMT, OP_LMH>(e, c.xn, c.emb, lm_rows, 0, nullptr);
  }
  hipLaunchKernelGGL(op_commit_kernel, dim3(1), dim3(ILL_WG_THREADS), 0, s, e->args, (const uint64_t*)c.amax, e->vocab / OP_BN, c.kvswz);
}

void op_seq_fmt(ill_engine* e, int M, int lm_rows) {
  if (e->fmt == 2) op_seq<2>(e, M, lm_rows);
  else if (e->fmt == 1) op_seq<1>(e, M, lm_rows);
  else op_seq<0>(e, M, lm_rows);
}

int op_launch(ill_engine* e, int M, int lm_rows) {
  HCK(hipEventRecord(e->ev0, e->stream));
  op_seq_fmt(e, M, lm_rows);
  HCK(hipGetLastError());
  HCK(hipEventRecord(e->ev1, e->stream));
  return 0;
}

}  // namespace

extern "C" {

const char* ill_last_error(void) { return g_err.c_str(); }

int ill_create(const char* path, int max_context, int max_pass, int max_steps, ill_engine** out) {
  if (!path || !out) return fail(ILL_E_ARG, "null argument");
  *out = nullptr;
  if (max_context < 64 || max_steps < 1) return fail(ILL_E_ARG, "bad sizes");
  if (max_pass < 1 || max_pass > ILL_MAXT) max_pass = ILL_MAXT;
  Mapped m;
  {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(ILL_E_FILE, "cannot open %s", path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
      close(fd);
      return fail(ILL_E_FILE, "cannot stat %s", path);
    }
    m.len = (size_t)sb.st_size;
    if (m.len < (size_t)kHeader) {
      close(fd);
      return fail(ILL_E_FILE, "%s: bad size %zu", path, m.len);
    }
    m.base = mmap(nullptr, m.len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m.base == MAP_FAILED) {
      m.base = nullptr;
      return fail(ILL_E_FILE, "mmap failed for %s", path);
    }
  }
  const uint8_t* base = (const uint8_t*)m.base;
  uint32_t hdr[4];
  memcpy(hdr, base, 16);
  if (hdr[0] != kMagic) return fail(ILL_E_FILE, "%s: not an instantllm model", path);
  if (hdr[1] != 1) return fail(ILL_E_FILE, "%s: unsupported version %u", path, hdr[1]);
  const int fmt = (int)hdr[2], count = (int)hdr[3];
  if (fmt < 0 || fmt > 2) return fail(ILL_E_FILE, "%s: unknown weight format %d", path, fmt);
  if (count < 16 || (count - 4) % 12 || 16 + (size_t)count * 16 > (size_t)kHeader) return fail(ILL_E_FILE, "%s: tensor table mismatch", path);
  const int layers = (count - 4) / 12;
  if (layers > ILL_MAXLAYERS) return fail(ILL_E_FILE, "%s: %d layers (max %d)", path, layers, ILL_MAXLAYERS);
  std::vector<uint64_t> tab(2 * (size_t)count);
  memcpy(tab.data(), base + 16, tab.size() * 8);
  auto off = [&](int id) { return tab[2 * id]; };
  auto size = [&](int id) { return tab[2 * id + 1]; };
  for (int id = 0; id < count; id++)
    if (size(id) && off(id) + size(id) > m.len) return fail(ILL_E_FILE, "%s: tensor %d out of range", path, id);
  auto need = [&](int id, size_t bytes) { return size(id) == bytes; };
  // matrix [rows][K]: q4 codes + (scale, min) per 64; q8 int8 + f16 scale per group
  // (32 or 64, read from the file, the same for every matrix); f16 values
  int q8g = 0;
  auto mat_ok = [&](int idw, int ids, int rows, int K) -> bool {
    if (fmt == 2) return need(idw, (size_t)rows * K / 2) && need(ids, (size_t)rows * (K / 64) * 4);
    if (fmt == 1) {
      if (!need(idw, (size_t)rows * K) || size(ids) == 0 || size(ids) % ((size_t)2 * rows)) return false;
      const size_t ng = size(ids) / 2 / rows;
      if (K % ng) return false;
      const int g = (int)(K / ng);
      if (g != 32 && g != 64) return false;
      if (q8g && q8g != g) return false;
      q8g = g;
      return true;
    }
    return need(idw, (size_t)rows * K * 2);
  };
  const int vocab = (int)(fmt == 2 ? size(0) * 2 / ILL_H : (fmt == 1 ? size(0) / ILL_H : size(0) / (2 * ILL_H)));
  if (vocab < 128 || vocab % 128 || !mat_ok(0, 1, vocab, ILL_H) || !need(2, ILL_H * 4))
    return fail(ILL_E_FILE, "%s: bad embedding tensors", path);
  for (int l = 0; l < layers; l++) {
    const int b = 3 + 12 * l;
    if (!need(b + 0, ILL_H * 4) || !mat_ok(b + 1, b + 2, ILL_QKV, ILL_H) || !need(b + 3, ILL_QKV * 4) ||
        !mat_ok(b + 4, b + 5, ILL_H, ILL_H) || !need(b + 6, ILL_H * 4) || !mat_ok(b + 7, b + 8, 2 * ILL_FF, ILL_H) ||
        !mat_ok(b + 9, b + 10, ILL_H, ILL_FF))
      return fail(ILL_E_FILE, "%s: layer %d tensor sizes do not match the model shape (format %d)", path, l, fmt);
  }

  ill_engine* e = new ill_engine();
  e->path = path;
  e->fmt = fmt;
  e->q8g = q8g ? q8g : 64;
  e->layers = layers;
  e->vocab = vocab;
  e->maxctx = (max_context + 63) / 64 * 64;
  e->maxpass = max_pass;
  e->maxsteps = max_steps;
  auto cleanup = [&](int rc) {
    ill_destroy(e);
    return rc;
  };

  // ---- device weight layout: one allocation, every tensor 256-byte aligned
  const size_t qkvW = (size_t)ILL_QKV * ILL_H / 2, qkvS = (size_t)ILL_QKV / 16 * ILL_KST * 128;
  const size_t oW = (size_t)ILL_H * ILL_H / 2, oS = (size_t)ILL_NH * ILL_NOT * 64;
  const size_t guW = (size_t)2 * ILL_FF * ILL_H / 2, guS = (size_t)2 * ILL_FF / 16 * ILL_KST * 128;
  const size_t dW = (size_t)ILL_H * ILL_FF / 2, dS = (size_t)ILL_NGU * ILL_NOT * 64;
  const size_t embW = (size_t)vocab * ILL_H / 2, embS = (size_t)vocab / 16 * ILL_KST * 128;
  size_t per_layer = al256(qkvW) + al256(qkvS) + al256(oW) + al256(oS) + al256(guW) + al256(guS) + al256(dW) + al256(dS) +
                     al256(ILL_QKV * 4) + 2 * al256(ILL_H * 4);
  size_t total = al256(embW) + al256(embS) + al256(ILL_H * 4) + per_layer * layers;
  std::vector<uint8_t> host(total);
  size_t cur = 0;
  auto take = [&](size_t n) {
    const size_t o = cur;
    cur += al256(n);
    return o;
  };
  std::vector<int> ident;
  // embedding / lm_head
  const size_t o_embW = take(embW), o_embS = take(embS), o_fn = take(ILL_H * 4);
  if (fmt == 2) {
    ident.resize(vocab);
    for (int i = 0; i < vocab; i++) ident[i] = i;
    repack_rows(base + off(0), (const uint32_t*)(base + off(1)), ILL_H, ident, host.data() + o_embW, (uint32_t*)(host.data() + o_embS));
    memcpy(host.data() + o_fn, base + off(2), ILL_H * 4);
  }
  struct LO { size_t qkvW, qkvS, oW, oS, guW, guS, dW, dS, b, ln1, ln2; };
  std::vector<LO> lo(layers);
  std::vector<int> rows_qkv(ILL_QKV), rows_o(ILL_H), rows_gu(2 * ILL_FF);
  for (int i = 0; i < ILL_QKV; i++) rows_qkv[i] = i;
  for (int i = 0; i < ILL_H; i++) rows_o[i] = i;
  // gate/up: unit block ub, tile k (0-3 gate, 4-7 up), row n -> unit 64 ub + 16 (k % 4) + n;
  // .ill row of gate unit u = 4 (u / 2) + u % 2, of up unit u = 4 (u / 2) + 2 + u % 2.
  for (int ub = 0; ub < ILL_NGU; ub++)
    for (int k = 0; k < 8; k++)
      for (int n = 0; n < 16; n++) {
        const int u = 64 * ub + 16 * (k & 3) + n;
        rows_gu[(ub * 8 + k) * 16 + n] = 4 * (u / 2) + (k >= 4 ? 2 : 0) + (u & 1);
      }
  for (int l = 0; l < layers; l++) {
    const int b = 3 + 12 * l;
    LO& L = lo[l];
    L.qkvW = take(qkvW); L.qkvS = take(qkvS); L.oW = take(oW); L.oS = take(oS);
    L.guW = take(guW); L.guS = take(guS); L.dW = take(dW); L.dS = take(dS);
    L.b = take(ILL_QKV * 4); L.ln1 = take(ILL_H * 4); L.ln2 = take(ILL_H * 4);
    if (fmt != 2) continue;   // the persistent pass kernel runs q4 models only
    repack_rows(base + off(b + 1), (const uint32_t*)(base + off(b + 2)), ILL_H, rows_qkv, host.data() + L.qkvW, (uint32_t*)(host.data() + L.qkvS));
    repack_split(base + off(b + 4), (const uint32_t*)(base + off(b + 5)), ILL_H, host.data() + L.oW, (uint32_t*)(host.data() + L.oS));
    repack_rows(base + off(b + 7), (const uint32_t*)(base + off(b + 8)), ILL_H, rows_gu, host.data() + L.guW, (uint32_t*)(host.data() + L.guS));
    repack_split(base + off(b + 9), (const uint32_t*)(base + off(b + 10)), ILL_FF, host.data() + L.dW, (uint32_t*)(host.data() + L.dS));
    memcpy(host.data() + L.b, base + off(b + 3), ILL_QKV * 4);
    memcpy(host.data() + L.ln1, base + off(b + 0), ILL_H * 4);
    memcpy(host.data() + L.ln2, base + off(b + 6), ILL_H * 4);
  }

  if (hipSetDevice(0) != hipSuccess) return cleanup(fail(ILL_E_HIP, "no HIP device"));
  int maxb = 0, maxb1 = 0;
  if (hipFuncSetAttribute((const void*)ill_pass_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, ill_stage_bytes(1)) != hipSuccess ||
      hipFuncSetAttribute((const void*)ill_pass_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize, ill_stage_bytes(4)) != hipSuccess ||
      hipFuncSetAttribute((const void*)ill_pass_kernel<16>, hipFuncAttributeMaxDynamicSharedMemorySize, ill_stage_bytes(16)) != hipSuccess)
    return cleanup(fail(ILL_E_HIP, "cannot raise the pass kernel's LDS limit to %d B", ill_stage_bytes(1)));
  int maxb4 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&maxb, ill_pass_kernel<16>, ILL_WG_THREADS, ill_stage_bytes(16)) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&maxb1, ill_pass_kernel<1>, ILL_WG_THREADS, ill_stage_bytes(1)) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&maxb4, ill_pass_kernel<4>, ILL_WG_THREADS, ill_stage_bytes(4)) != hipSuccess ||
      maxb < 1 || maxb1 < 1 || maxb4 < 1)
    return cleanup(fail(ILL_E_HIP, "pass kernel cannot be resident (occupancy %d / %d / %d)", maxb1, maxb4, maxb));
  maxb = std::min(std::min(maxb, maxb1), maxb4);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return cleanup(fail(ILL_E_HIP, "hipGetDeviceProperties failed"));
  if (prop.multiProcessorCount * maxb < ILL_WG)
    return cleanup(fail(ILL_E_HIP, "device has %d CUs x %d: the persistent pass needs %d resident workgroups", prop.multiProcessorCount, maxb, ILL_WG));
  if (hipStreamCreate(&e->stream) != hipSuccess) return cleanup(fail(ILL_E_HIP, "hipStreamCreate failed"));
  if (hipEventCreate(&e->ev0) != hipSuccess || hipEventCreate(&e->ev1) != hipSuccess) return cleanup(fail(ILL_E_HIP, "hipEventCreate failed"));
  if (hipMalloc(&e->dweights, total) != hipSuccess) return cleanup(fail(ILL_E_HIP, "weights allocation failed (%zu B)", total));
  if (hipMemcpy(e->dweights, host.data(), total, hipMemcpyHostToDevice) != hipSuccess) return cleanup(fail(ILL_E_HIP, "weights upload failed"));
  host.clear();
  host.shrink_to_fit();
  uint8_t* D = e->dweights;
  e->W.wemb = D + o_embW;
  e->W.semb = (const uint32_t*)(D + o_embS);
  e->W.fnorm = (const float*)(D + o_fn);
  e->W.vocab = vocab;
  e->W.layers = layers;
  e->W.fmt = fmt;
  e->hlayers.resize(layers);
  for (int l = 0; l < layers; l++) {
    IllLayerW& w = e->hlayers[l];
    const LO& L = lo[l];
    w.wqkv = D + L.qkvW; w.sqkv = (const uint32_t*)(D + L.qkvS);
    w.wo = D + L.oW; w.so = (const uint32_t*)(D + L.oS);
    w.wgu = D + L.guW; w.sgu = (const uint32_t*)(D + L.guS);
    w.wd = D + L.dW; w.sd = (const uint32_t*)(D + L.dS);
    w.bqkv = (const float*)(D + L.b); w.ln1 = (const float*)(D + L.ln1); w.ln2 = (const float*)(D + L.ln2);
  }
  // ---- layer-by-layer path: the .ill matrices as stored (row-major, file row orders)
  {
    std::vector<size_t> place(count, 0);
    size_t otot = 0;
    for (int id = 0; id < count; id++) {
      place[id] = otot;
      otot += al256(size(id));
    }
    // q8 / f16: W_o head-major for the attention-fused O projection (OpLayerW::oh)
    const bool ohead = fmt != 2;
    const int es = fmt == 0 ? 2 : 1, nchk = 64 * es / 16, qg = e->q8g;
    const size_t ohw = (size_t)ILL_NH * nchk * ILL_H * 16, ohs = (size_t)ILL_NH * ILL_H * 4;
    std::vector<size_t> p_ohw(layers, 0), p_ohs(layers, 0);
    if (ohead)
      for (int l = 0; l < layers; l++) {
        p_ohw[l] = otot;
        otot += al256(ohw);
        p_ohs[l] = otot;
        otot += al256(ohs);
      }
    std::vector<uint8_t> oh(otot);
    for (int id = 0; id < count; id++)
      if (size(id)) memcpy(oh.data() + place[id], base + off(id), size(id));
    // q8 / f16: the matrices tiled for the GEMM kernels (op_wt_off / op_st_off, ill_ops.h)
    auto tile = [&](int idw, int ids, int N, int K) {
      const int es = fmt == 0 ? 2 : 1, unit = 16 / es;
      if (N % 128 || K % 64 || size(idw) < (size_t)N * K * es || (fmt == 1 && size(ids) < (size_t)N * (K / qg) * 2)) return false;
      const uint8_t* src = base + off(idw);
      uint8_t* dst = oh.data() + place[idw];
      for (int r = 0; r < N; r++)
        for (int k = 0; k < K; k += unit) memcpy(dst + op_wt_off(r, k, K, es), src + ((size_t)r * K + k) * es, 16);
      if (fmt == 1) {
        const uint16_t* ss = (const uint16_t*)(base + off(ids));
        uint16_t* sd = (uint16_t*)(oh.data() + place[ids]);
        for (int r = 0; r < N; r++)
          for (int g = 0; g < K / qg; g++) sd[op_st_off(r, g * qg, K, qg)] = ss[(size_t)r * (K / qg) + g];
      }
      return true;
    };
    if (fmt != 2) {
      bool tiled = tile(0, 1, vocab, ILL_H);
      for (int l = 0; l < layers && tiled; l++) {
        const int b = 3 + 12 * l;
        tiled = tile(b + 1, b + 2, ILL_QKV, ILL_H) && tile(b + 4, b + 5, ILL_H, ILL_H) && tile(b + 7, b + 8, 2 * ILL_FF, ILL_H) &&
                tile(b + 9, b + 10, ILL_H, ILL_FF);
      }
      if (!tiled) return cleanup(fail(ILL_E_FILE, "a q8 / f16 matrix does not have the expected shape"));
    }
    if (ohead)
      for (int l = 0; l < layers; l++) {
        const int b = 3 + 12 * l;
        if (size(b + 4) < (size_t)ILL_H * ILL_H * es || (fmt == 1 && size(b + 5) < (size_t)ILL_H * (ILL_H / qg) * 2))
          return cleanup(fail(ILL_E_FILE, "layer %d: W_o tensors too small", l));
        const uint8_t* wsrc = base + off(b + 4);
        const uint16_t* ssrc = (const uint16_t*)(base + off(b + 5));
        for (int h = 0; h < ILL_NH; h++)
          for (int i = 0; i < nchk; i++)
            for (int r = 0; r < ILL_H; r++)
              memcpy(oh.data() + p_ohw[l] + (((size_t)h * nchk + i) * ILL_H + r) * 16, wsrc + ((size_t)r * ILL_H + 64 * h) * es + 16 * i, 16);
        if (fmt == 1)
          for (int h = 0; h < ILL_NH; h++)
            for (int r = 0; r < ILL_H; r++) {
              const uint32_t v = (uint32_t)ssrc[(size_t)r * (ILL_H / qg) + (64 * h) / qg] |
                                 ((uint32_t)ssrc[(size_t)r * (ILL_H / qg) + (64 * h + 32) / qg] << 16);
              memcpy(oh.data() + p_ohs[l] + ((size_t)h * ILL_H + r) * 4, &v, 4);
            }
      }
    if (hipMalloc(&e->oweights, otot) != hipSuccess) return cleanup(fail(ILL_E_HIP, "weights allocation failed (%zu B)", otot));
    if (hipMemcpy(e->oweights, oh.data(), otot, hipMemcpyHostToDevice) != hipSuccess) return cleanup(fail(ILL_E_HIP, "weights upload failed"));
    uint8_t* O = e->oweights;
    auto mk = [&](int idw, int ids, int rows, int K) {
      OpMat m;
      m.w = O + place[idw];
      m.s = (const uint16_t*)(O + place[ids]);
      m.N = rows;
      m.K = K;
      m.qg = e->q8g;
      return m;
    };
    e->holayers.resize(layers);
    for (int l = 0; l < layers; l++) {
      const int b = 3 + 12 * l;
      OpLayerW& w = e->holayers[l];
      w.qkv = mk(b + 1, b + 2, ILL_QKV, ILL_H);
      w.o = mk(b + 4, b + 5, ILL_H, ILL_H);
      w.oh = w.o;
      if (ohead) {
        w.oh.w = O + p_ohw[l];
        w.oh.s = (const uint16_t*)(O + p_ohs[l]);
      }
      w.gu = mk(b + 7, b + 8, 2 * ILL_FF, ILL_H);
      w.d = mk(b + 9, b + 10, ILL_H, ILL_FF);
      w.bqkv = (const float*)(O + place[b + 3]);
      w.ln1 = (const float*)(O + place[b + 0]);
      w.ln2 = (const float*)(O + place[b + 6]);
    }
    e->octx.emb = mk(0, 1, vocab, ILL_H);
    e->octx.fnorm = (const float*)(O + place[2]);
  }
  auto dalloc = [&](void** p, size_t bytes) {
    if (hipMalloc(p, bytes) != hipSuccess) return false;
    return hipMemset(*p, 0, bytes) == hipSuccess;
  };
  const size_t kvb = (size_t)layers * ILL_NKV * e->maxctx * 64 * 2;
  e->acc_bytes = (size_t)2 * layers * ILL_NKIND * 16 * ILL_ACC_ROW * 8;
  bool ok = dalloc((void**)&e->dlayers, sizeof(IllLayerW) * layers) && dalloc((void**)&e->st, 64) && dalloc((void**)&e->ctl, 64) &&
            dalloc((void**)&e->ptoks, ILL_OP_MAXM * 4) && dalloc((void**)&e->tree, ILL_TR_INTS * 4) &&
            dalloc((void**)&e->rope, (size_t)(e->maxctx + 16) * 32 * 8) && dalloc((void**)&e->kc, kvb) && dalloc((void**)&e->vt, kvb) &&
            dalloc((void**)&e->acc, e->acc_bytes) &&
            dalloc((void**)&e->lmp, (size_t)ILL_WG * 16 * 2 * 8) && dalloc((void**)&e->pub, (size_t)ILL_PUB_WORDS * 8) &&
            dalloc((void**)&e->part, (size_t)ILL_PART_WORDS * 16) &&
            dalloc((void**)&e->logits, (size_t)16 * vocab * 4) &&
            dalloc((void**)&e->out_dev, (size_t)max_steps * 4);
  ok = ok && dalloc((void**)&e->dolayers, sizeof(OpLayerW) * layers) && dalloc((void**)&e->octx.x, (size_t)ILL_OP_MAXM * ILL_H * 4) &&
       dalloc((void**)&e->octx.xn, (size_t)ILL_OP_MAXM * ILL_H * 2) && dalloc((void**)&e->octx.q, (size_t)ILL_OP_MAXM * ILL_H * 4) &&
       dalloc((void**)&e->octx.ao, (size_t)ILL_OP_MAXM * ILL_H * 2) && dalloc((void**)&e->octx.h, (size_t)ILL_OP_MAXM * ILL_FF * 2) &&
       dalloc((void**)&e->octx.amax, (size_t)(vocab / OP_BN) * 16 * 8) && dalloc((void**)&e->opart, ILL_OP_PART_BYTES);
  if (!ok) return cleanup(fail(ILL_E_HIP, "device buffer allocation failed"));
  if (hipMemcpy(e->dolayers, e->holayers.data(), sizeof(OpLayerW) * layers, hipMemcpyHostToDevice) != hipSuccess)
    return cleanup(fail(ILL_E_HIP, "layer table upload failed"));
  if (hipHostMalloc((void**)&e->out_host, (size_t)max_steps * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&e->spec_host, 2 * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&e->stop_host, 4, hipHostMallocCoherent) != hipSuccess)
    return cleanup(fail(ILL_E_HIP, "pinned token buffer allocation failed"));
  e->spec_host[0] = e->spec_host[1] = 0;
  *(volatile int32_t*)e->stop_host = 0;
  if (!dalloc((void**)&e->prompt, (4 + ILL_OB_MAX) * 4)) return cleanup(fail(ILL_E_HIP, "prompt buffer allocation failed"));
  for (int i = 0; i < max_steps; i++) e->out_host[i] = -1;
  if (hipMemcpy(e->dlayers, e->hlayers.data(), sizeof(IllLayerW) * layers, hipMemcpyHostToDevice) != hipSuccess)
    return cleanup(fail(ILL_E_HIP, "layer table upload failed"));
  {
    // RoPE table: angle = pos * theta^(-2i/64) in float64, cos/sin rounded once to fp32
    // (tools/reference/qwen_ref.py:118-127).
    std::vector<float2> r((size_t)(e->maxctx + 16) * 32);
    for (int p = 0; p < e->maxctx + 16; p++)
      for (int i = 0; i < 32; i++) {
        const double inv = 1.0 / std::pow(1000000.0, (double)(2 * i) / 64.0);
        const double ang = (double)p * inv;
        r[(size_t)p * 32 + i] = make_float2((float)std::cos(ang), (float)std::sin(ang));
      }
    if (hipMemcpy(e->rope, r.data(), r.size() * 8, hipMemcpyHostToDevice) != hipSuccess) return cleanup(fail(ILL_E_HIP, "rope upload failed"));
  }
  {
    IllCtl c{};
    c.epoch = 1;
    if (hipMemcpy(e->ctl, &c, sizeof c, hipMemcpyHostToDevice) != hipSuccess) return cleanup(fail(ILL_E_HIP, "ctl upload failed"));
    IllState s{};
    s.maxctx = e->maxctx;
    s.maxsteps = max_steps;
    s.eos0 = 151645;
    s.eos1 = 151643;
    s.nver = 1;
    s.tspec = 1;
    s.done = 1;   // idle until a request sets the state
    if (hipMemcpy(e->st, &s, sizeof s, hipMemcpyHostToDevice) != hipSuccess) return cleanup(fail(ILL_E_HIP, "state upload failed"));
  }
  IllPassArgs& a = e->args;
  a.W = e->W;
  a.L = e->dlayers;
  a.L0 = e->hlayers[0];
  a.st = e->st;
  a.ctl = e->ctl;
  a.ptoks = e->ptoks;
  a.tree = e->tree;
  a.rope = e->rope;
  a.kc = e->kc;
  a.vt = e->vt;
  a.acc = e->acc;
  a.lmp = e->lmp;
  a.pub = e->pub;
  a.part = e->part;
  a.logits = e->logits;
  a.out_dev = e->out_dev;
  a.out_host = e->out_host;
  a.spec_host = e->spec_host;
  a.stop_host = e->stop_host;
  a.prompt = e->prompt;
  a.ngram = nullptr;
  a.maxctx = e->maxctx;
  a.maxsteps = max_steps;
  OpCtx& oc = e->octx;
  oc.L = e->dolayers;
  oc.st = e->st;
  oc.ctl = e->ctl;
  oc.ptoks = e->ptoks;
  oc.tree = e->tree;
  oc.rope = e->rope;
  oc.kc = e->kc;
  oc.vt = e->vt;
  oc.kvswz = e->fmt != 2 ? 1 : 0;
  oc.logits = e->logits;
  oc.maxctx = e->maxctx;
  oc.layers = layers;
  oc.vocab = vocab;
  if (hipDeviceSynchronize() != hipSuccess) return cleanup(fail(ILL_E_HIP, "device sync failed"));
  *out = e;
  return ILL_OK;
}

int ill_destroy(ill_engine* e) {
  if (!e) return ILL_OK;
  if (e->stream) hipStreamSynchronize(e->stream);
  if (e->gexec) hipGraphExecDestroy(e->gexec);
  if (e->graph) hipGraphDestroy(e->graph);
  void* bufs[] = {e->dweights, e->dlayers, e->st, e->ctl, e->ptoks, e->tree, e->rope, e->kc, e->vt, e->acc,
                  e->lmp, e->pub, e->part, e->logits, e->out_dev, e->args.trace, e->oweights, e->dolayers, e->octx.x, e->octx.xn,
                  e->octx.q, e->octx.ao, e->octx.h, e->octx.amax, e->opart, e->dtab, e->dtflg, e->dreq};
  for (void* p : bufs)
    if (p) hipFree(p);
  if (e->out_host) hipHostFree(e->out_host);
  if (e->spec_host) hipHostFree(e->spec_host);
  if (e->stop_host) hipHostFree(e->stop_host);
  if (e->prompt) hipFree(e->prompt);
  if (e->ngram) hipFree(e->ngram);
  delete e->ild;
  if (e->ev0) hipEventDestroy(e->ev0);
  if (e->ev1) hipEventDestroy(e->ev1);
  if (e->stream) hipStreamDestroy(e->stream);
  delete e;
  return ILL_OK;
}

int ill_vocab(const ill_engine* e) { return e ? e->vocab : ILL_E_ARG; }
int ill_layers(const ill_engine* e) { return e ? e->layers : ILL_E_ARG; }
int ill_format(const ill_engine* e) { return e ? e->fmt : ILL_E_ARG; }

int ill_set_state(ill_engine* e, const int32_t state[16]) {
  if (!e || !state) return fail(ILL_E_ARG, "null argument");
  IllState s;
  memcpy(&s, state, sizeof s);
  if (s.maxctx != e->maxctx) s.maxctx = e->maxctx;
  if (s.maxsteps > e->maxsteps || s.maxsteps < 1) return fail(ILL_E_ARG, "maxsteps %d outside 1..%d", s.maxsteps, e->maxsteps);
  if (s.pos < 0 || s.pos >= e->maxctx) return fail(ILL_E_ARG, "pos %d outside the context", s.pos);
  if (!s.done) {
    // a live state must let the commits record into out_tokens and a pass of up to 16 rows
    // at pos stay inside the context (the device keeps both true after every commit)
    if (s.step < 0 || s.step >= s.maxsteps) return fail(ILL_E_ARG, "step %d outside 0..%d", s.step, s.maxsteps - 1);
    if (s.n < 1 || s.n > e->maxctx) return fail(ILL_E_ARG, "n %d outside 1..%d", s.n, e->maxctx);
    if (s.pos + ILL_MAXT > e->maxctx) return fail(ILL_E_ARG, "pos %d leaves no room for a pass in the context %d", s.pos, e->maxctx);
  }
  if (s.learned && !e->ild) return fail(ILL_E_ARG, "the State asks for the learned drafter but no table is loaded");
  HCK(hipMemcpyAsync(e->st, &s, sizeof s, hipMemcpyHostToDevice, e->stream));
  // the learned drafter's shape: trees of learned_tree drafts, else chains of tspec rows
  const int32_t tb = s.learned && e->learned_tree > 0 ? std::min(e->learned_tree, ILL_MAXT - 1) : 0;
  HCK(hipMemcpyAsync(&e->ctl->tree_b, &tb, 4, hipMemcpyHostToDevice, e->stream));
  HCK(hipStreamSynchronize(e->stream));
  // a new State starts a new request: the device is idle, so no commit reads the word now
  __atomic_store_n(e->stop_host, 0, __ATOMIC_SEQ_CST);
  e->pos_hint = s.pos;
  e->learned_active = s.learned != 0;
  return ILL_OK;
}

int ill_stop(ill_engine* e) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  __atomic_store_n(e->stop_host, 1, __ATOMIC_SEQ_CST);
  return ILL_OK;
}

int ill_get_state(ill_engine* e, int32_t state[16]) {
  if (!e || !state) return fail(ILL_E_ARG, "null argument");
  IllState s;
  const int rc = read_state(e, &s);
  if (rc) return rc;
  memcpy(state, &s, sizeof s);
  return ILL_OK;
}

int ill_prefill(ill_engine* e, const int32_t* toks, int n, int write_logits) {
  if (!e || !toks || n < 1) return fail(ILL_E_ARG, "bad prefill arguments");
  touch_cache(e);
  IllState s;
  int rc = read_state(e, &s);
  if (rc) return rc;
  if (s.done) return fail(ILL_E_ARG, "state is done: set the state before a prefill");
  if (s.pos + n + 16 > e->maxctx) return fail(ILL_E_ARG, "prompt of %d tokens at pos %d exceeds the context %d", n, s.pos, e->maxctx);
  for (int i = 0; i < n; i++)
    if (toks[i] < 0 || toks[i] >= e->vocab) return fail(ILL_E_ARG, "token %d out of range", toks[i]);
  int pos = s.pos;
  // encodePrefill commits through k_commit_spec when speculation is on (Engine.swift:588-601):
  // the State's tspec > 1 makes the prompt's commit draft the first verify pass
  const int fin = s.tspec > 1 ? 2 : 1;
  if (e->fmt != 2 || n > 16) {   // layer-by-layer path, chunks of up to ILL_OP_MAXM rows
    for (int c0 = 0; c0 < n; c0 += ILL_OP_MAXM) {
      const int rows = n - c0 < ILL_OP_MAXM ? n - c0 : ILL_OP_MAXM;
      const bool last = c0 + rows == n;
      HCK(hipMemcpyAsync(e->ptoks, toks + c0, rows * 4, hipMemcpyHostToDevice, e->stream));
      if ((rc = write_pos_n(e, pos, rows))) return rc;
      if ((rc = set_ctl(e, ILL_MODE_ROWS, rows, 0, last ? 1 : 0, last ? write_logits : 0, last ? fin : 0))) return rc;
      e->pos_hint = pos;
      if ((rc = op_launch(e, rows, last ? 1 : 0))) return rc;
      if (last && fin == 2 && (rc = launch_draft(e))) return rc;
      pos += rows;
      HCK(hipStreamSynchronize(e->stream));
    }
    if (write_logits) e->logits_rows_valid = 1;
    e->pos_hint = s.pos + n;
    return check_err(e);
  }
  for (int c0 = 0; c0 < n; c0 += 16) {
    const int rows = n - c0 < 16 ? n - c0 : 16;
    const bool last = c0 + rows == n;
    HCK(hipMemcpyAsync(e->ptoks, toks + c0, rows * 4, hipMemcpyHostToDevice, e->stream));
    if ((rc = write_pos_n(e, pos, rows))) return rc;
    if (last) rc = set_ctl(e, ILL_MODE_ROWS, rows, rows - 1, 1, write_logits, fin);
    else rc = set_ctl(e, ILL_MODE_ROWS, rows, 0, 0, 0, 0);
    if (rc) return rc;
    if ((rc = launch(e, pass_T(rows)))) return rc;
    if (last && fin == 2 && (rc = launch_draft(e))) return rc;
    pos += rows;
    // the staging copies above read host memory asynchronously: keep `toks` alive
    HCK(hipStreamSynchronize(e->stream));
  }
  if (write_logits) e->logits_rows_valid = 0;
  e->pos_hint = s.pos + n;
  if ((rc = check_err(e))) return rc;
  if (write_logits) {
    // the last row's logits sit at row (rows - 1); move them to row 0 for ill_read_logits
    const int rows = (n - 1) % 16 + 1;
    if (rows != 1) HCK(hipMemcpy(e->logits, e->logits + (size_t)(rows - 1) * e->vocab, (size_t)e->vocab * 4, hipMemcpyDeviceToDevice));
    e->logits_rows_valid = 1;
  }
  return ILL_OK;
}

int ill_decode_step(ill_engine* e, int write_logits) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  touch_cache(e);
  int rc = set_ctl(e, ILL_MODE_DECODE, 1, 0, 1, write_logits, 1);
  if (rc) return rc;
  if ((rc = e->fmt == 2 ? launch(e, 1) : op_launch(e, 1, 1))) return rc;
  e->pos_hint++;
  if ((rc = check_err(e))) return rc;
  if (write_logits) e->logits_rows_valid = 1;
  return ILL_OK;
}

int ill_verify_pass(ill_engine* e, int rows, const int32_t* tree, const int32_t* toks, int write_logits) {
  if (!e || rows < 1 || rows > 16) return fail(ILL_E_ARG, "rows must be 1..16");
  touch_cache(e);
  int32_t tk[16];
  if (tree) {
    if (tree[0] != rows) return fail(ILL_E_ARG, "tree[0] = %d but rows = %d", tree[0], rows);
    for (int i = 1; i < rows; i++) {
      const int p = tree[ILL_TR_PARENT + i];
      if (p < 0 || p >= i) return fail(ILL_E_ARG, "tree parent[%d] = %d must be in 0..%d", i, p, i - 1);
      if (tree[ILL_TR_DEPTH + i] != tree[ILL_TR_DEPTH + p] + 1) return fail(ILL_E_ARG, "tree depth[%d] inconsistent with its parent", i);
    }
    if (tree[ILL_TR_DEPTH] != 0) return fail(ILL_E_ARG, "tree root depth must be 0");
    for (int i = 0; i < rows; i++) tk[i] = tree[ILL_TR_TOK + i];
  } else {
    if (!toks) return fail(ILL_E_ARG, "chain pass needs toks");
    for (int i = 0; i < rows; i++) tk[i] = toks[i];
  }
  for (int i = 0; i < rows; i++)
    if (tk[i] < 0 || tk[i] >= e->vocab) return fail(ILL_E_ARG, "token %d out of range", tk[i]);
  IllState s;
  int rc = read_state(e, &s);
  if (rc) return rc;
  if (s.done) return fail(ILL_E_ARG, "state is done");
  if (s.pos + 16 > e->maxctx) return fail(ILL_E_ARG, "pass exceeds the context");
  HCK(hipMemcpyAsync(e->ptoks, tk, rows * 4, hipMemcpyHostToDevice, e->stream));
  if (tree) HCK(hipMemcpyAsync(e->tree, tree, ILL_TR_INTS * 4, hipMemcpyHostToDevice, e->stream));
  if ((rc = write_pos_n(e, s.pos, rows))) return rc;
  if ((rc = set_ctl(e, tree ? ILL_MODE_TREE : ILL_MODE_ROWS, rows, 0, rows, write_logits, 2))) return rc;
  e->pos_hint = s.pos;
  if ((rc = e->fmt == 2 ? launch(e, pass_T(rows)) : op_launch(e, rows, rows))) return rc;
  if ((rc = launch_draft(e))) return rc;   // the next pass's drafts (ill_spec_pass continues from here)
  e->pos_hint = s.pos + 1;   // at least the root is accepted
  if ((rc = check_err(e))) return rc;
  if (write_logits) e->logits_rows_valid = rows;
  return ILL_OK;
}

// ---- speculative decoding with on-device drafting (k_commit_spec, Shaders.swift:246-418) ----
int ill_load_ngram(ill_engine* e, const void* table, int64_t bytes) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  HCK(hipStreamSynchronize(e->stream));
  if (!table || bytes == 0) {
    if (e->ngram) HCK(hipFree(e->ngram));
    e->ngram = nullptr;
  } else {
    if (bytes != (int64_t)ILL_NG_SLOTS * 16) return fail(ILL_E_ARG, "n-gram table of %lld bytes (expected %d)", (long long)bytes, ILL_NG_SLOTS * 16);
    // every occupied slot {u64 key, i32 next, u16 count, u16 total} must name a token of
    // this model's vocabulary: the drafter embeds it in the next pass
    const uint32_t* sl = (const uint32_t*)table;
    for (int i = 0; i < ILL_NG_SLOTS; i++) {
      const uint32_t* q = sl + 4 * i;
      if ((q[0] | q[1]) && (int32_t)q[2] >= 0 && (int32_t)q[2] < e->vocab) continue;
      if (q[0] | q[1]) return fail(ILL_E_ARG, "n-gram slot %d: next token %d outside the vocabulary", i, (int32_t)q[2]);
    }
    if (!e->ngram) HCK(hipMalloc((void**)&e->ngram, (size_t)bytes));
    HCK(hipMemcpy(e->ngram, table, (size_t)bytes, hipMemcpyHostToDevice));
  }
  e->args.ngram = (const uint4*)e->ngram;
  drop_graph(e);   // captured passes hold the table pointer
  return ILL_OK;
}

int ill_set_prompt(ill_engine* e, const int32_t* toks, int n) {
  if (!e || (n > 0 && !toks) || n < 0) return fail(ILL_E_ARG, "bad prompt");
  int32_t buf[4 + ILL_OB_MAX] = {0};
  const int np = n < ILL_OB_MAX ? n : ILL_OB_MAX;
  for (int i = n - np; i < n; i++)   // the drafter proposes these tokens
    if (toks[i] < 0 || toks[i] >= e->vocab) return fail(ILL_E_ARG, "prompt token %d out of range", toks[i]);
  buf[0] = np;
  for (int i = 0; i < np; i++) buf[4 + i] = toks[n - np + i];
  HCK(hipMemcpyAsync(e->prompt, buf, sizeof buf, hipMemcpyHostToDevice, e->stream));
  HCK(hipStreamSynchronize(e->stream));
  return ILL_OK;
}

namespace {
// write_logits of the next launch only (a speculative pass takes its rows and commit from
// the control block the previous commit wrote)
int set_wlog(ill_engine* e, int wlog) {
  e->hctl.write_logits = wlog;
  HCK(hipMemcpyAsync(&e->ctl->write_logits, &e->hctl.write_logits, 4, hipMemcpyHostToDevice, e->stream));
  return 0;
}
}  // namespace

int ill_spec_pass(ill_engine* e, int write_logits) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  touch_cache(e);
  IllState s;
  int rc = read_state(e, &s);
  if (rc) return rc;
  if (s.done) return ILL_OK;   // a stopped request: nothing to do (the device would early-exit)
  IllCtl c;
  HCK(hipMemcpy(&c, e->ctl, sizeof c, hipMemcpyDeviceToHost));
  if (c.commit != 2 || c.draft || c.nrows < 1 || c.nrows > ILL_MAXT)
    return fail(ILL_E_ARG, "no drafted pass pending (prefill with the State's tspec > 1, or run a verify pass, first)");
  if ((rc = set_wlog(e, write_logits))) return rc;
  e->pos_hint = s.pos;
  if ((rc = e->fmt == 2 ? launch(e, pass_T(c.nrows)) : op_launch(e, c.nrows, c.nrows))) return rc;
  if ((rc = launch_draft(e))) return rc;
  if ((rc = check_err(e))) return rc;
  if (write_logits) e->logits_rows_valid = c.nrows;
  return ILL_OK;
}

int ill_capture_spec(ill_engine* e, int npasses) {
  if (!e || npasses < 1) return fail(ILL_E_ARG, "bad pass count");
  drop_graph(e);
  // every pass has at most the State's tspec rows: the smallest instantiation that holds them
  IllState s;
  if (int rc = read_state(e, &s)) return rc;
  const int T = pass_T(std::max(2, std::min(s.tspec, ILL_MAXT)));
  HCK(hipStreamSynchronize(e->stream));
  HCK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
  for (int i = 0; i < npasses; i++) {
    enqueue_pass(e, T);
    enqueue_draft(e);
  }
  HCK(hipStreamEndCapture(e->stream, &e->graph));
  HCK(hipGraphInstantiate(&e->gexec, e->graph, nullptr, nullptr, 0));
  e->graph_steps = npasses;
  e->graph_spec = true;
  e->graph_T = T;
  e->graph_learned = e->learned_active;
  return ILL_OK;
}

namespace {
// generate_spec's graph of `npasses` chained passes on the T-row instantiation (cached per
// T, drafting kernel and pass count), then launched: the passes take their rows from the
// device, so every pending pass must hold at most T rows.
int launch_spec_graph(ill_engine* e, int T, int npasses) {
  ill_engine::SpecGraph& g = e->sg[T == 1 ? 0 : (T == 4 ? 1 : 2)];
  if (!g.x || g.steps != npasses || g.learned != e->learned_active) {
    if (g.x) HCK(hipGraphExecDestroy(g.x));
    if (g.g) HCK(hipGraphDestroy(g.g));
    g = ill_engine::SpecGraph{};
    HCK(hipStreamSynchronize(e->stream));
    HCK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < npasses; i++) {
      enqueue_pass(e, T);
      enqueue_draft(e);
    }
    HCK(hipStreamEndCapture(e->stream, &g.g));
    HCK(hipGraphInstantiate(&g.x, g.g, nullptr, nullptr, 0));
    g.steps = npasses;
    g.learned = e->learned_active;
  }
  if (int rc = set_wlog(e, 0)) return rc;
  if (int rc = count_passes(e, npasses)) return rc;
  HCK(hipGraphLaunch(g.x, e->stream));
  return 0;
}

// one pass of generate_spec on the T-row instantiation and its drafting, launched directly
// (a pass after a change of shape, or one of a shape not yet judged)
int launch_spec_one(ill_engine* e, int T) {
  if (int rc = set_wlog(e, 0)) return rc;
  if (int rc = count_passes(e, 1)) return rc;
  enqueue_pass(e, T);
  enqueue_draft(e);
  HCK(hipGetLastError());
  return 0;
}
}  // namespace

int ill_capture_steps(ill_engine* e, int nsteps) {
  if (!e || nsteps < 1) return fail(ILL_E_ARG, "bad step count");
  drop_graph(e);
  e->graph_spec = false;
  HCK(hipStreamSynchronize(e->stream));
  HCK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
  const int base = e->pos_hint;
  for (int i = 0; i < nsteps; i++) {
    e->pos_hint = base + i;
    if (e->fmt == 2) hipLaunchKernelGGL(ill_pass_kernel<1>, dim3(ILL_WG), dim3(ILL_WG_THREADS), ill_stage_bytes(1), e->stream, e->args);
    else op_seq_fmt(e, 1, 1);
  }
  e->pos_hint = base;
  HCK(hipStreamEndCapture(e->stream, &e->graph));
  HCK(hipGraphInstantiate(&e->gexec, e->graph, nullptr, nullptr, 0));
  e->graph_steps = nsteps;
  return ILL_OK;
}

int ill_launch_graph(ill_engine* e) { return ill_launch_graph_logits(e, 0); }

int ill_launch_graph_logits(ill_engine* e, int write_logits) {
  if (!e || !e->gexec) return fail(ILL_E_ARG, "no captured graph");
  touch_cache(e);
  int rc = e->graph_spec ? set_wlog(e, write_logits ? 1 : 0) : set_ctl(e, ILL_MODE_DECODE, 1, 0, 1, write_logits ? 1 : 0, 1);
  if (rc) return rc;
  if ((rc = count_passes(e, e->graph_steps))) return rc;
  HCK(hipGraphLaunch(e->gexec, e->stream));
  e->pos_hint += e->graph_steps;
  if (write_logits) e->logits_rows_valid = 1;
  return ILL_OK;
}

int ill_sync(ill_engine* e) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  return check_err(e);
}

const int32_t* ill_out_tokens(ill_engine* e) { return e ? e->out_host : nullptr; }

int ill_reset_out_tokens(ill_engine* e) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  HCK(hipStreamSynchronize(e->stream));
  for (int i = 0; i < e->maxsteps; i++) e->out_host[i] = -1;
  return ILL_OK;
}

int ill_read_logits(ill_engine* e, int row, float* out) {
  if (!e || !out || row < 0 || row >= 16) return fail(ILL_E_ARG, "bad logits row");
  HCK(hipStreamSynchronize(e->stream));
  HCK(hipMemcpy(out, e->logits + (size_t)row * e->vocab, (size_t)e->vocab * 4, hipMemcpyDeviceToHost));
  return ILL_OK;
}

// reference cache layout [layer][kvh][npos][64]; the engine keeps K and V in blocks of 64
// slots, in rows (q4) or swizzled (q8 / f16): kv_k_off / kv_v_off, ill_common.h.
int ill_kv_copy_out(ill_engine* e, int npos, uint16_t* k, uint16_t* v) {
  if (!e || !k || !v || npos < 0 || npos > e->maxctx) return fail(ILL_E_ARG, "bad kv copy");
  HCK(hipStreamSynchronize(e->stream));
  const size_t per = (size_t)e->maxctx * 64;
  const bool swz = e->fmt != 2;
  std::vector<uint16_t> kt(per), vtt(per);
  for (int lh = 0; lh < e->layers * ILL_NKV; lh++) {
    HCK(hipMemcpy(kt.data(), e->kc + lh * per, per * 2, hipMemcpyDeviceToHost));
    HCK(hipMemcpy(vtt.data(), e->vt + lh * per, per * 2, hipMemcpyDeviceToHost));
    for (int p = 0; p < npos; p++)
      for (int d = 0; d < 64; d++) {
        k[((size_t)lh * npos + p) * 64 + d] = kt[kv_k_off(p, d, swz)];
        v[((size_t)lh * npos + p) * 64 + d] = vtt[kv_v_off(p, d, swz)];
      }
  }
  return ILL_OK;
}

int ill_kv_copy_in(ill_engine* e, int npos, const uint16_t* k, const uint16_t* v) {
  if (!e || !k || !v || npos < 0 || npos > e->maxctx) return fail(ILL_E_ARG, "bad kv copy");
  touch_cache(e);
  HCK(hipStreamSynchronize(e->stream));
  const size_t per = (size_t)e->maxctx * 64;
  const bool swz = e->fmt != 2;
  std::vector<uint16_t> kt(per), vtt(per);
  for (int lh = 0; lh < e->layers * ILL_NKV; lh++) {
    HCK(hipMemcpy(kt.data(), e->kc + lh * per, per * 2, hipMemcpyDeviceToHost));
    HCK(hipMemcpy(vtt.data(), e->vt + lh * per, per * 2, hipMemcpyDeviceToHost));
    for (int p = 0; p < npos; p++)
      for (int d = 0; d < 64; d++) {
        kt[kv_k_off(p, d, swz)] = k[((size_t)lh * npos + p) * 64 + d];
        vtt[kv_v_off(p, d, swz)] = v[((size_t)lh * npos + p) * 64 + d];
      }
    HCK(hipMemcpy(e->kc + lh * per, kt.data(), per * 2, hipMemcpyHostToDevice));
    HCK(hipMemcpy(e->vt + lh * per, vtt.data(), per * 2, hipMemcpyHostToDevice));
  }
  return ILL_OK;
}

}  // extern "C"

namespace {
// Marks the passes of one generate call as its own (they keep the prefix cache).
struct GenScope {
  ill_engine* e;
  explicit GenScope(ill_engine* x) : e(x) { e->in_generate = true; }
  ~GenScope() { e->in_generate = false; }
};

// Engine.swift:929-933: positions 0 .. common - 1 already hold this prompt's K/V (at least
// one token is always prefilled, for its logits).
int prefix_reuse(ill_engine* e, const int32_t* toks, int ntok) {
  int common = 0;
  const int lim = std::min((int)e->cached.size(), ntok);
  while (common < lim && e->cached[common] == toks[common]) common++;
  if (common == ntok) common--;
  e->last_prefill = ntok - common;
  e->cached.clear();   // set again when the call completes
  return common;
}

// Engine.swift:1029-1031: K/V are valid for the prompt and every generated token but the
// last one.
void set_cached(ill_engine* e, const int32_t* toks, int ntok, const int32_t* out, int nout) {
  e->cached.assign(toks, toks + ntok);
  for (int i = 0; i + 1 < nout; i++) e->cached.push_back(out[i]);
}

// Engine.prefixKey (Engine.swift:790-794): the model file's size and modification time and
// the context length; a saved prefix loads only into the same model file and context.
bool prefix_key(const ill_engine* e, uint64_t key[5]) {
  struct stat sb;
  if (stat(e->path.c_str(), &sb) != 0) return false;
  key[0] = 0x31564B4C4C49ull;
  key[1] = (uint64_t)sb.st_size;
  key[2] = (uint64_t)sb.st_mtim.tv_sec;
  key[3] = (uint64_t)sb.st_mtim.tv_nsec;
  key[4] = (uint64_t)e->maxctx;
  return true;
}
}  // namespace

extern "C" {

int ill_truncate_cache(ill_engine* e, int n) {
  if (!e || n < 0) return fail(ILL_E_ARG, "bad truncate arguments");
  if ((int)e->cached.size() > n) e->cached.resize((size_t)n);
  return ILL_OK;
}

int ill_prefix_info(ill_engine* e, int* cached, int* last_prefill) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  if (cached) *cached = (int)e->cached.size();
  if (last_prefill) *last_prefill = e->last_prefill;
  return ILL_OK;
}

// Engine.savePrefix (Engine.swift:796-811): [key 5 x u64][n u64][n x i32 tokens] then K and V
// of positions 0..n-1 as [layer][kv head][n][64] f16 (the reference's cache layout).
int ill_save_prefix(ill_engine* e, const char* path, const int32_t* toks, int n) {
  if (!e || !path || !toks || n < 1) return fail(ILL_E_ARG, "bad prefix arguments");
  if (n > (int)e->cached.size() || !std::equal(toks, toks + n, e->cached.begin()))
    return fail(ILL_E_ARG, "the %d tokens are not a prefix of the cached tokens (%zu)", n, e->cached.size());
  uint64_t key[6];
  if (!prefix_key(e, key)) return fail(ILL_E_FILE, "cannot stat the model file %s", e->path.c_str());
  key[5] = (uint64_t)n;
  const size_t per = (size_t)e->layers * ILL_NKV * n * 64;
  std::vector<uint16_t> k(per), v(per);
  e->in_generate = true;   // reading the cache keeps it
  int rc = ill_kv_copy_out(e, n, k.data(), v.data());
  e->in_generate = false;
  if (rc) return rc;
  const std::string tmp = std::string(path) + ".tmp";
  FILE* f = fopen(tmp.c_str(), "wb");
  if (!f) return fail(ILL_E_FILE, "cannot write %s", tmp.c_str());
  const bool ok = fwrite(key, 8, 6, f) == 6 && fwrite(toks, 4, (size_t)n, f) == (size_t)n &&
                  fwrite(k.data(), 2, per, f) == per && fwrite(v.data(), 2, per, f) == per;
  if (fclose(f) != 0 || !ok || rename(tmp.c_str(), path) != 0) {
    remove(tmp.c_str());
    return fail(ILL_E_FILE, "writing %s failed", path);
  }
  return ILL_OK;
}

// Engine.loadPrefix (Engine.swift:813-838): loads a prefix saved for this model file and
// context; returns its tokens (the generate prefix cache then starts from them).
int ill_load_prefix(ill_engine* e, const char* path, int32_t* toks, int max_toks, int* n_out) {
  if (!e || !path || !n_out) return fail(ILL_E_ARG, "bad prefix arguments");
  *n_out = 0;
  FILE* f = fopen(path, "rb");
  if (!f) return fail(ILL_E_FILE, "cannot open %s", path);
  uint64_t hdr[6], key[5];
  bool ok = fread(hdr, 8, 6, f) == 6 && prefix_key(e, key);
  for (int i = 0; ok && i < 5; i++) ok = hdr[i] == key[i];
  const uint64_t n = ok ? hdr[5] : 0;
  ok = ok && n > 0 && n < (uint64_t)e->maxctx;
  if (ok && toks && (int)n > max_toks) ok = false;
  std::vector<int32_t> t(ok ? n : 0);
  const size_t per = (size_t)e->layers * ILL_NKV * n * 64;
  std::vector<uint16_t> k(ok ? per : 0), v(ok ? per : 0);
  ok = ok && fread(t.data(), 4, n, f) == n && fread(k.data(), 2, per, f) == per && fread(v.data(), 2, per, f) == per &&
       fgetc(f) == EOF;
  fclose(f);
  if (!ok) return fail(ILL_E_FILE, "%s is not a prefix saved for this model file and context", path);
  int rc = ill_kv_copy_in(e, (int)n, k.data(), v.data());
  if (rc) return rc;
  e->cached = t;
  if (toks) std::copy(t.begin(), t.end(), toks);
  *n_out = (int)n;
  return ILL_OK;
}

int ill_generate(ill_engine* e, const int32_t* toks, int ntok, int max_new, int chunk, int32_t* out, int* n_out, float* logits_out) {
  return ill_generate_cb(e, toks, ntok, max_new, chunk, out, n_out, logits_out, nullptr, nullptr);
}

int ill_generate_cb(ill_engine* e, const int32_t* toks, int ntok, int max_new, int chunk, int32_t* out, int* n_out,
                    float* logits_out, ill_token_fn on_token, void* user) {
  if (!e || !toks || ntok < 1 || max_new < 1 || !out || !n_out) return fail(ILL_E_ARG, "bad generate arguments");
  if (max_new > e->maxsteps) return fail(ILL_E_ARG, "max_new %d > max_steps %d", max_new, e->maxsteps);
  // Engine.swift:934 (tokens + maxNew <= maxContext), with the 16-slot margin of a pass
  if (ntok + max_new + ILL_MAXT > e->maxctx)
    return fail(ILL_E_ARG, "prompt of %d tokens + %d new exceeds the context %d (less a 16-slot pass margin)", ntok, max_new, e->maxctx);
  if (chunk < 1) chunk = 1;
  *n_out = 0;
  GenScope scope(e);
  int rc;
  if ((rc = ill_reset_out_tokens(e))) return rc;
  const int common = prefix_reuse(e, toks, ntok);
  int32_t s[16] = {0};
  s[0] = common;
  s[1] = ntok - common;
  s[4] = e->maxctx;
  s[5] = max_new;
  s[6] = 151645;
  s[7] = 151643;
  s[8] = 1;
  s[9] = 1;
  if ((rc = ill_set_state(e, s))) return rc;
  if ((rc = ill_prefill(e, toks + common, ntok - common, logits_out != nullptr))) return rc;
  if (logits_out && (rc = ill_read_logits(e, 0, logits_out))) return rc;
  if ((e->graph_spec || e->graph_steps != chunk) && (rc = ill_capture_steps(e, chunk))) return rc;
  volatile const int32_t* ot = e->out_host;
  int got = 0, encoded = 1;
  bool stopped = false;
  while (!stopped && got < max_new) {
    if (encoded < max_new && encoded - got <= chunk) {
      if ((rc = ill_launch_graph(e))) return rc;
      encoded += chunk;
      continue;
    }
    const int t = ot[got];
    if (t < 0) {
      // a finished stream with no new token means the device stopped (or failed)
      if (hipStreamQuery(e->stream) == hipSuccess && ot[got] < 0) {
        if ((rc = check_err(e))) return rc;
        if (encoded >= max_new) break;
      }
      continue;
    }
    got++;
    if (t == 151645 || t == 151643) break;
    out[(*n_out)++] = t;
    if (on_token && !on_token(t, user)) {
      // Engine.swift:1021-1036: the caller stopped the request; steps still queued leave
      // at once (the next commit reads the stop word and sets the State's done flag)
      stopped = true;
      if (got < encoded) ill_stop(e);
    }
  }
  HCK(hipStreamSynchronize(e->stream));
  if ((rc = check_err(e))) return rc;
  set_cached(e, toks, ntok, out, *n_out);
  return ILL_OK;
}

int ill_generate_spec(ill_engine* e, const int32_t* toks, int ntok, int max_new, int rows, int chunk, int adaptive,
                      int32_t* out, int* n_out, int32_t* stats) {
  if (!e || !toks || ntok < 1 || max_new < 1 || !out || !n_out) return fail(ILL_E_ARG, "bad generate arguments");
  // Requests with a drafter context use the learned drafter (Engine.swift:950-956): chains
  // of learned_T rows or trees of learned_tree drafts; others the commit's own drafting
  const bool learned = e->draft_ctx_ready && e->use_learned && e->ild;
  const int treeb = learned && e->learned_tree > 0 ? std::min(e->learned_tree, ILL_MAXT - 1) : 0;
  if (learned) rows = treeb > 0 ? treeb + 1 : e->learned_T;
  if (rows < 2 || rows > ILL_MAXT) return fail(ILL_E_ARG, "rows per speculative pass %d outside 2..%d", rows, ILL_MAXT);
  if (max_new > e->maxsteps) return fail(ILL_E_ARG, "max_new %d > max_steps %d", max_new, e->maxsteps);
  if (ntok + max_new + ILL_MAXT > e->maxctx)
    return fail(ILL_E_ARG, "prompt of %d tokens + %d new exceeds the context %d (less a 16-slot pass margin)", ntok, max_new, e->maxctx);
  if (chunk < 1) chunk = 1;
  e->draft_ctx_ready = false;
  *n_out = 0;
  int rc;
  GenScope scope(e);
  if ((rc = ill_reset_out_tokens(e)) || (rc = ill_set_prompt(e, toks, ntok))) return rc;
  e->spec_host[0] = e->spec_host[1] = 0;
  const int common = prefix_reuse(e, toks, ntok);
  int32_t s[16] = {0};
  s[0] = common;
  s[1] = ntok - common;
  s[4] = e->maxctx;
  s[5] = max_new;
  s[6] = 151645;
  s[7] = 151643;
  s[8] = 1;
  s[9] = rows;   // tspec: the prompt's commit drafts the first pass
  s[14] = learned ? 1 : 0;
  if ((rc = ill_set_state(e, s))) return rc;
  int cur_tree = treeb;
  HCK(hipMemcpyAsync(&e->ctl->tree_b, &cur_tree, 4, hipMemcpyHostToDevice, e->stream));
  if ((rc = ill_prefill(e, toks + common, ntok - common, 0))) return rc;
  // Pass shapes (Engine.nextPassShape, Engine.swift:888-898, with thresholds from this
  // engine's pass costs, which grow with the kernel's row count: about 340 us for 1 row,
  // 800 us for 4 and 860 us for 16, plus the drafting, up to 250 us for a learned tree): a
  // pass of 1 + r tokens beats plain decoding when r >= 1.6 accepted drafts (4 rows) or
  // r >= 2.3 (16 rows with a drafted tree). Level 0 is the configured shape, kept while
  // r >= 2.4 over the last four passes of that shape; level 1 a 4-row chain (3 drafts), back
  // to level 0 at r >= 2.2, kept at r >= 1.6; level 2 one-row passes without drafts (a
  // decode step's cost), left for a 4-row probe after `probe_gap` passes. A level is judged
  // on the passes that hold rows drafted at its shape: after two of them, or after one that
  // accepted no draft, and at most one of them is in flight before that verdict. The
  // configured shape falls straight to one-row passes when fewer than one draft per pass is
  // accepted; every probe that fails doubles the gap to the next (16 .. 128 passes), a probe
  // that pays resets it. A pass holds the rows drafted after the pass before it, so the pass
  // after a change of shape runs on the instantiation of the previous shape, the rest on
  // their own; a change to one-row passes cuts that pass to its first row instead.
  int level = 0, probe_gap = 16;
  bool probing = false;
  int lv_first = 0;         // the first pass holding rows drafted at this level's shape
  std::vector<int> samp;    // samp[d]: accepted drafts once d passes after the prefill committed
  int encoded = 0;          // passes enqueued after the prefill
  volatile const int32_t* ot = e->out_host;
  volatile const int32_t* sp = e->spec_host;
  // passes committed after the prefill (-1 before the prompt's commit), with the accepted
  // count read first: the commit stores it after the pass count, so a pairing is at worst
  // stale, and refreshed by the next read while the pass count stands
  auto observe = [&]() -> int {
    const int acc = sp[1];
    const int d = sp[0] - 1;
    if (d < 0) return -1;
    if ((int)samp.size() <= d) samp.resize(d + 1, acc);
    samp[d] = acc;
    return d;
  };
  // the level for the next pass and whether its shape has been judged
  auto next_level = [&](int done, bool& judged) -> int {
    judged = true;
    if (!adaptive) return 0;
    if (level == 2) return encoded - lv_first >= probe_gap ? 1 : 2;
    const int n = done - lv_first;
    judged = n >= 2 || (n == 1 && samp[done] == samp[lv_first]);
    if (!judged) return level;
    const int d0 = std::max(lv_first, done - 4);
    const double rate = (double)(samp[done] - samp[d0]) / (double)(done - d0);
    if (level == 0) return rate >= 2.4 ? 0 : (rows > 4 && rate >= 1.0 ? 1 : (rate >= 1.6 ? 0 : 2));
    return rate >= 2.2 ? 0 : (rate >= 1.6 ? 1 : 2);
  };
  int cur_rows = rows;
  int drafted_rows = rows;   // the most rows the next pass can hold (the prompt's commit drafted it)
  int got = 0;   // tokens read
  while (got < max_new) {
    const int done = observe();
    // keep at most one chunk of passes ahead of the committed ones (Engine.swift:991-1008);
    // every pass commits at least one token, so max_new passes always suffice
    if (encoded < max_new && encoded - done <= chunk) {
      bool judged;
      const int lv = next_level(done, judged);
      if (lv != level) {
        if (level == 2 && lv == 1) probing = true;
        else if (probing) {   // the probe's verdict
          probe_gap = lv == 2 ? std::min(2 * probe_gap, 128) : 16;
          probing = false;
        }
        level = lv;
        lv_first = encoded + 1;
        judged = level == 2;
        const int want_rows = level == 0 ? rows : (level == 1 ? std::min(rows, 4) : 1);
        const int want_tree = level == 0 ? treeb : 0;
        if (want_rows != cur_rows || want_tree != cur_tree) {   // ordered after the passes before it
          cur_rows = want_rows;
          cur_tree = want_tree;
          HCK(hipMemcpyAsync(&e->st->tspec, &cur_rows, 4, hipMemcpyHostToDevice, e->stream));
          HCK(hipMemcpyAsync(&e->ctl->tree_b, &cur_tree, 4, hipMemcpyHostToDevice, e->stream));
        }
        if (level == 2 && drafted_rows > 1) {   // the pending pass, cut to its first row
          hipLaunchKernelGGL(ill_trunc_kernel, dim3(1), dim3(64), 0, e->stream, e->args);
          HCK(hipGetLastError());
          drafted_rows = 1;
        }
      }
      // an unjudged shape has at most one of its passes in flight (the host sees a commit
      // while its drafting still runs, and launches the next pass behind it)
      if (judged || encoded <= std::max(done, lv_first)) {
        if (pass_T(drafted_rows) != pass_T(cur_rows) || !judged) {
          if ((rc = launch_spec_one(e, pass_T(drafted_rows)))) return rc;
          encoded++;
        } else {
          if ((rc = launch_spec_graph(e, pass_T(cur_rows), chunk))) return rc;
          encoded += chunk;
        }
        drafted_rows = cur_rows;
        continue;
      }
    }
    const int t = ot[got];
    if (t < 0) {
      // an idle stream with no new token: the device stopped (or every pass is spent)
      if (hipStreamQuery(e->stream) == hipSuccess && ot[got] < 0 && observe() == done) {
        IllState st;
        if ((rc = check_err(e)) || (rc = read_state(e, &st))) return rc;
        if (st.done || encoded >= max_new) break;
      }
      continue;
    }
    got++;
    if (t == 151645 || t == 151643) break;
    out[(*n_out)++] = t;
  }
  HCK(hipStreamSynchronize(e->stream));
  if ((rc = check_err(e))) return rc;
  set_cached(e, toks, ntok, out, *n_out);
  if (stats) {
    IllState st;
    if ((rc = read_state(e, &st))) return rc;
    stats[0] = st.passes;
    stats[1] = st.accepted;
  }
  return ILL_OK;
}

// ---- learned drafter (ILDraft.swift, Engine.swift:865-913) -------------------------------
struct ill_ildraft {
  illd::Table t;
};

ill_ildraft* ill_ildraft_open(const char* path) {
  if (!path) {
    fail(ILL_E_ARG, "null path");
    return nullptr;
  }
  ill_ildraft* d = new ill_ildraft();
  const std::string err = illd::load(d->t, path);
  if (!err.empty()) {
    delete d;
    fail(ILL_E_FILE, "%s", err.c_str());
    return nullptr;
  }
  return d;
}

void ill_ildraft_close(ill_ildraft* d) { delete d; }

int ill_ildraft_prepare(ill_ildraft* d, const int32_t* prompt, int n, const char* text, ill_encode_fn encode, void* user) {
  if (!d || n < 0 || (n > 0 && !prompt)) return fail(ILL_E_ARG, "bad drafter context");
  illd::prepare(d->t, prompt, n, text, encode, user);
  return ILL_OK;
}

int64_t ill_ildraft_request(const ill_ildraft* d, void* out, int64_t bytes) {
  if (!d) return fail(ILL_E_ARG, "null drafter");
  if (out && bytes >= (int64_t)sizeof(IllDraftReq)) memcpy(out, &d->t.req, sizeof(IllDraftReq));
  return (int64_t)sizeof(IllDraftReq);
}

int ill_load_ildraft(ill_engine* e, const char* path) {
  if (!e || !path) return fail(ILL_E_ARG, "null argument");
  illd::Table* t = new illd::Table();
  const std::string err = illd::load(*t, path);
  if (!err.empty()) {
    delete t;
    return fail(ILL_E_FILE, "%s", err.c_str());
  }
  // the new table goes into buffers of its own first: on any failure the engine keeps no
  // drafter (never a pointer to freed memory) and the new table is released
  uint8_t* tab = nullptr;
  int rc = ILL_OK;
  const illd::HashIndex hx = illd::build_index(*t);
  if (hx.bytes.empty()) {
    delete t;
    return fail(ILL_E_FILE, "learned drafter table too large to index (a section of more than 2^27 entries)");
  }
  const size_t hoff = (t->blob.size() + 255) & ~(size_t)255;   // the indexes after the table
  if (hipStreamSynchronize(e->stream) != hipSuccess || hipMalloc((void**)&tab, hoff + hx.bytes.size()) != hipSuccess ||
      hipMemcpy(tab, t->blob.data(), t->blob.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(tab + hoff, hx.bytes.data(), hx.bytes.size(), hipMemcpyHostToDevice) != hipSuccess ||
      (!e->dtflg && hipMalloc((void**)&e->dtflg, ILD_VOCAB) != hipSuccess) ||
      hipMemcpy(e->dtflg, t->tflg.data(), ILD_VOCAB, hipMemcpyHostToDevice) != hipSuccess ||
      (!e->dreq && hipMalloc((void**)&e->dreq, sizeof(IllDraftReq)) != hipSuccess) ||
      hipMemset(e->dreq, 0, sizeof(IllDraftReq)) != hipSuccess)
    rc = fail(ILL_E_HIP, "learned drafter table upload failed");
  drop_graph(e);   // captured drafting kernels hold the old table's pointers
  if (e->dtab) (void)hipFree(e->dtab);
  e->dtab = nullptr;
  delete e->ild;
  e->ild = nullptr;
  e->dargs = IllDraftArgs{};
  e->draft_ctx_ready = false;
  if (rc != ILL_OK) {
    if (tab) (void)hipFree(tab);
    delete t;
    return rc;
  }
  e->dtab = tab;
  e->ild = t;
  e->dargs = illd::device_args(*t, e->dtab, e->dtflg, e->dreq, hx, e->dtab + hoff);
  return ILL_OK;
}

int ill_set_draft_context(ill_engine* e, const int32_t* prompt, int n, const char* text, ill_encode_fn encode, void* user) {
  if (!e || n < 0 || (n > 0 && !prompt)) return fail(ILL_E_ARG, "bad drafter context");
  if (!e->ild) return ILL_OK;   // no table: the request drafts with the commit's own drafter
  illd::prepare(*e->ild, prompt, n, text, encode, user);
  HCK(hipStreamSynchronize(e->stream));
  HCK(hipMemcpy(e->dreq, &e->ild->req, sizeof(IllDraftReq), hipMemcpyHostToDevice));
  e->draft_ctx_ready = true;
  return ILL_OK;
}

int ill_set_learned(ill_engine* e, int use, int chain_rows, int tree_budget) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  if (chain_rows < 2 || chain_rows > ILL_MAXT) return fail(ILL_E_ARG, "chain rows %d outside 2..%d", chain_rows, ILL_MAXT);
  if (tree_budget < 0) return fail(ILL_E_ARG, "negative tree budget");
  e->use_learned = use != 0;
  e->learned_T = chain_rows;
  e->learned_tree = tree_budget;
  return ILL_OK;
}

int ill_pending_pass(ill_engine* e, int32_t info[4], int32_t toks[16], int32_t tree[65]) {
  if (!e || !info) return fail(ILL_E_ARG, "null argument");
  IllCtl c;
  HCK(hipStreamSynchronize(e->stream));
  HCK(hipMemcpy(&c, e->ctl, sizeof c, hipMemcpyDeviceToHost));
  info[0] = c.mode;
  info[1] = c.nrows;
  info[2] = c.commit;
  info[3] = c.draft;
  if (toks) HCK(hipMemcpy(toks, e->ptoks, 16 * 4, hipMemcpyDeviceToHost));
  if (tree) HCK(hipMemcpy(tree, e->tree, ILL_TR_INTS * 4, hipMemcpyDeviceToHost));
  return ILL_OK;
}

int ill_time_graph(ill_engine* e, int iters, float* ms) {
  if (!e || !e->gexec || iters < 1 || !ms) return fail(ILL_E_ARG, "bad timing arguments");
  hipEvent_t a, b;
  HCK(hipEventCreate(&a));
  HCK(hipEventCreate(&b));
  int rc = e->graph_spec ? set_wlog(e, 0) : set_ctl(e, ILL_MODE_DECODE, 1, 0, 1, 0, 1);
  if (rc) return rc;
  if ((rc = count_passes(e, iters * e->graph_steps))) return rc;
  HCK(hipEventRecord(a, e->stream));
  for (int i = 0; i < iters; i++) HCK(hipGraphLaunch(e->gexec, e->stream));
  HCK(hipEventRecord(b, e->stream));
  HCK(hipEventSynchronize(b));
  HCK(hipEventElapsedTime(ms, a, b));
  hipEventDestroy(a);
  hipEventDestroy(b);
  return check_err(e);
}

int ill_trace_enable(ill_engine* e, int on) {
  if (!e) return fail(ILL_E_ARG, "null engine");
  HCK(hipStreamSynchronize(e->stream));
  // a captured graph holds the trace pointer in its kernel arguments: it is dropped
  // whenever the trace buffer comes or goes (capture again after toggling)
  if ((on != 0) != (e->args.trace != nullptr)) drop_graph(e);
  if (on && !e->args.trace) {
    void* p = nullptr;
    HCK(hipMalloc(&p, (size_t)ILL_WG * ILL_TRACE_SLOTS * 8));
    HCK(hipMemset(p, 0, (size_t)ILL_WG * ILL_TRACE_SLOTS * 8));
    e->args.trace = (uint64_t*)p;
  } else if (!on && e->args.trace) {
    HCK(hipFree(e->args.trace));
    e->args.trace = nullptr;
  }
  return ILL_OK;
}

int ill_trace_read(ill_engine* e, uint64_t* out, int* slots) {
  if (!e || !out || !slots) return fail(ILL_E_ARG, "null argument");
  if (!e->args.trace) return fail(ILL_E_ARG, "trace is off");
  HCK(hipStreamSynchronize(e->stream));
  HCK(hipMemcpy(out, e->args.trace, (size_t)ILL_WG * ILL_TRACE_SLOTS * 8, hipMemcpyDeviceToHost));
  *slots = ILL_TRACE_SLOTS;
  return ILL_OK;
}

int ill_last_pass_ms(ill_engine* e, float* ms) {
  if (!e || !ms) return fail(ILL_E_ARG, "null argument");
  HCK(hipEventSynchronize(e->ev1));
  HCK(hipEventElapsedTime(ms, e->ev0, e->ev1));
  return ILL_OK;
}

}  // extern "C"

// ---- stand-alone q4 GEMV (microbench of the decode step's matrix-vector product) -------
// Scratch of the allocation-free entry point ill_gemv_run_noalloc: the argmax keys
// [ILL_SCRATCH_KEYS] and, for callers that pass no y, the product itself (at most
// ILL_SCRATCH_YMAX rows). Each GPU holds its own copy of this array until the process ends;
// host code uses the per-device address from hipGetSymbolAddress (never the array's name).
// Every call on a GPU shares that GPU's copy, which keeps the last call's contents (the keys
// are cleared by a fill kernel at the start of each call): calls that overlap on one GPU
// race.
#define ILL_SCRATCH_KEYS 2
#define ILL_SCRATCH_YMAX 262144
static __device__ __align__(256) uint64_t scratch[ILL_SCRATCH_KEYS + ILL_SCRATCH_YMAX / 2];

namespace {
#define ILL_MAX_DEVICES 64
std::mutex g_scratch_mu;
uint64_t* g_scratch_dev[ILL_MAX_DEVICES] = {};

// Address of this GPU's scratch array (the current device), looked up once per device.
int scratch_for_current_device(uint64_t** out) {
  int dev = 0;
  HCK(hipGetDevice(&dev));
  if (dev < 0 || dev >= ILL_MAX_DEVICES) return fail(ILL_E_HIP, "device %d outside 0..%d", dev, ILL_MAX_DEVICES - 1);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    HCK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(ILL_E_HIP, "no device address for the scratch array");
    g_scratch_dev[dev] = (uint64_t*)p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}

__global__ void gemv_key_clear_kernel(uint64_t* key) {
  if (threadIdx.x < ILL_SCRATCH_KEYS) gst(key + threadIdx.x, (uint64_t)0);
}
__global__ void gemv_key_finish_kernel(const uint64_t* key, int32_t* amax) {
  if (threadIdx.x == 0) gst(amax, (int32_t)(0xFFFFFFFFu - (uint32_t)(gld(key) & 0xFFFFFFFFu)));
}
}  // namespace

extern "C" {

struct ill_gemv {
  int rows = 0, K = 0, nb = 0, bps = 1, ks = 1, copies = 0;
  std::vector<uint8_t*> w;
  std::vector<uint32_t*> s;
  float* x = nullptr;
  float* gamma = nullptr;
  float* y = nullptr;
  uint64_t* key = nullptr;
  uint64_t* scratch = nullptr;   // this GPU's scratch array (ill_gemv_run_noalloc)
  hipStream_t stream = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
};

int ill_gemv_destroy(ill_gemv* g) {
  if (!g) return ILL_OK;
  if (g->stream) hipStreamSynchronize(g->stream);
  for (auto p : g->w) hipFree(p);
  for (auto p : g->s) hipFree(p);
  hipFree(g->x);
  hipFree(g->gamma);
  hipFree(g->y);
  hipFree(g->key);
  if (g->e0) hipEventDestroy(g->e0);
  if (g->e1) hipEventDestroy(g->e1);
  if (g->stream) hipStreamDestroy(g->stream);
  delete g;
  return ILL_OK;
}

int ill_gemv_create(int rows, int K, const uint8_t* codes, const uint32_t* sb, int copies, ill_gemv** out) {
  if (!out) return fail(ILL_E_ARG, "null output handle");
  *out = nullptr;
  if (!codes || !sb || rows < 16 || rows % 16 || K < 128 || K % 128 || K > 64 * ILL_GEMV_MAXG || copies < 1)
    return fail(ILL_E_ARG, "gemv shape %d x %d (rows: multiple of 16; K: multiple of 128, <= %d), copies %d",
                rows, K, 64 * ILL_GEMV_MAXG, copies);
  ill_gemv* g = new ill_gemv();
  auto bad = [&](int rc) { ill_gemv_destroy(g); return rc; };
  g->rows = rows;
  g->K = K;
  g->nb = K / 128;
  g->copies = copies;
  const int ntile = rows / 16;
  // slices per tile: the most (at most one per wave) that still fit every tile of the matrix
  // in one round of the grid; one slice (whole tiles, one per wave) when even that does not
  int ks = 1;
  for (int k = std::min(g->nb, ILL_WAVES); k > 1; k--)
    if ((ntile + ILL_WAVES / k - 1) / (ILL_WAVES / k) <= ILL_WG) {
      ks = k;
      break;
    }
  int bps = (g->nb + ks - 1) / ks;
  if (bps > ILL_GEMV_MAXBPS) bps = ILL_GEMV_MAXBPS;
  g->bps = bps;
  g->ks = (g->nb + bps - 1) / bps;
  std::vector<int> order(rows);
  for (int i = 0; i < rows; i++) order[i] = i;
  std::vector<uint8_t> hw((size_t)ntile * g->nb * 1024);
  std::vector<uint32_t> hs((size_t)ntile * g->nb * 32);
  repack_rows(codes, sb, K, order, hw.data(), hs.data());
  if (hipSetDevice(0) != hipSuccess) return bad(fail(ILL_E_HIP, "no HIP device"));
  if (int rc = scratch_for_current_device(&g->scratch)) return bad(rc);
  for (int c = 0; c < copies; c++) {
    uint8_t* pw = nullptr;
    uint32_t* ps = nullptr;
    if (hipMalloc(&pw, hw.size()) != hipSuccess || hipMalloc(&ps, hs.size() * 4) != hipSuccess) {
      if (pw) hipFree(pw);
      return bad(fail(ILL_E_HIP, "weight copy %d allocation failed", c));
    }
    g->w.push_back(pw);
    g->s.push_back(ps);
    if (hipMemcpy(pw, hw.data(), hw.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ps, hs.data(), hs.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return bad(fail(ILL_E_HIP, "weight copy %d upload failed", c));
  }
  if (hipMalloc(&g->x, (size_t)K * 4) != hipSuccess || hipMalloc(&g->gamma, (size_t)K * 4) != hipSuccess ||
      hipMalloc(&g->y, (size_t)rows * 4) != hipSuccess ||
      hipMalloc(&g->key, 16) != hipSuccess)
    return bad(fail(ILL_E_HIP, "gemv buffer allocation failed"));
  if (hipStreamCreate(&g->stream) != hipSuccess || hipEventCreate(&g->e0) != hipSuccess || hipEventCreate(&g->e1) != hipSuccess)
    return bad(fail(ILL_E_HIP, "stream / event creation failed"));
  *out = g;
  return ILL_OK;
}

int ill_gemv_run(ill_gemv* g, const float* x, const float* gamma, int iters, float* y, int32_t* amax, float* us_per_iter) {
  if (!g || !x || iters < 1) return fail(ILL_E_ARG, "bad gemv run arguments");
  HCK(hipMemcpyAsync(g->x, x, (size_t)g->K * 4, hipMemcpyHostToDevice, g->stream));
  if (gamma) HCK(hipMemcpyAsync(g->gamma, gamma, (size_t)g->K * 4, hipMemcpyHostToDevice, g->stream));
  HCK(hipStreamSynchronize(g->stream));
  IllGemvArgs a{};
  a.x = g->x;
  a.gamma = gamma ? g->gamma : nullptr;
  a.rows = g->rows;
  a.K = g->K;
  a.bps = g->bps;
  a.ks = g->ks;
  // one kernel writes y and the argmax (keys alternate between two words, each launch
  // clearing the other one): with one slice every item is a whole tile, with several the
  // slices of a tile are summed in LDS by the workgroup that computed them
  if (amax) HCK(hipMemsetAsync(g->key, 0, 16, g->stream));
  a.y = g->y;
  a.key = amax ? g->key : nullptr;
  const int ntile = g->rows / 16;
  const int tpr = ILL_WAVES / g->ks;   // ks <= 8: bps <= 8 and K <= 64 * 128
  const int grid = std::min(ILL_WG, (ntile + tpr - 1) / tpr);
  int par = 0;
  auto one = [&](int c) -> int {
    a.w = g->w[c];
    a.s = g->s[c];
    a.par = par;
    if (g->ks == 1)
      hipLaunchKernelGGL(ill_gemv_q4_kernel, dim3(ILL_WG), dim3(ILL_WG_THREADS), 0, g->stream, a);
    else
      hipLaunchKernelGGL(ill_gemv_q4_tiles_kernel, dim3(grid), dim3(ILL_WG_THREADS), 0, g->stream, a);
    par ^= 1;
    HCK(hipGetLastError());
    return 0;
  };
  int rc = one(0);   // warm
  if (rc) return rc;
  HCK(hipEventRecord(g->e0, g->stream));
  for (int i = 0; i < iters; i++)
    if ((rc = one(i % g->copies))) return rc;
  HCK(hipEventRecord(g->e1, g->stream));
  HCK(hipEventSynchronize(g->e1));
  float ms = 0.f;
  HCK(hipEventElapsedTime(&ms, g->e0, g->e1));
  if (us_per_iter) *us_per_iter = ms * 1e3f / (float)iters;
  if (y) HCK(hipMemcpy(y, g->y, (size_t)g->rows * 4, hipMemcpyDeviceToHost));
  if (amax) {
    uint64_t k = 0;
    HCK(hipMemcpy(&k, g->key + (par ^ 1), 8, hipMemcpyDeviceToHost));
    *amax = (int32_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu));
  }
  return ILL_OK;
}

int ill_gemv_run_noalloc(ill_gemv* g, int copy, const float* x, const float* gamma, float* y, int32_t* amax, void* stream) {
  if (!g || !x) return fail(ILL_E_ARG, "null gemv or x");
  if (copy < 0 || copy >= g->copies) return fail(ILL_E_ARG, "weight copy %d outside 0..%d", copy, g->copies - 1);
  if (!y && !amax) return fail(ILL_E_ARG, "nothing to compute: pass y, argmax or both");
  if (!y && g->rows > ILL_SCRATCH_YMAX)
    return fail(ILL_E_ARG, "%d rows exceed the %d-row scratch: pass a y buffer", g->rows, ILL_SCRATCH_YMAX);
  hipStream_t st = stream ? (hipStream_t)stream : g->stream;
  IllGemvArgs a{};
  a.w = g->w[copy];
  a.s = g->s[copy];
  a.x = x;
  a.gamma = gamma;
  a.rows = g->rows;
  a.K = g->K;
  a.bps = g->bps;
  a.ks = g->ks;
  a.y = y ? y : (float*)(g->scratch + ILL_SCRATCH_KEYS);
  a.key = amax ? g->scratch : nullptr;
  a.par = 0;
  if (amax) hipLaunchKernelGGL(gemv_key_clear_kernel, dim3(1), dim3(64), 0, st, g->scratch);
  if (g->ks == 1) {
    hipLaunchKernelGGL(ill_gemv_q4_kernel, dim3(ILL_WG), dim3(ILL_WG_THREADS), 0, st, a);
  } else {
    const int tpr = ILL_WAVES / g->ks;
    const int grid = std::min(ILL_WG, (g->rows / 16 + tpr - 1) / tpr);
    hipLaunchKernelGGL(ill_gemv_q4_tiles_kernel, dim3(grid), dim3(ILL_WG_THREADS), 0, st, a);
  }
  if (amax) hipLaunchKernelGGL(gemv_key_finish_kernel, dim3(1), dim3(64), 0, st, (const uint64_t*)g->scratch, amax);
  HCK(hipGetLastError());
  return ILL_OK;
}

int ill_quantize_q4(const float* w, int64_t rows, int cols, uint8_t* packed, uint16_t* sb, int threads) {
  if (!w || !packed || !sb || rows < 1 || cols < 64 || cols % 64) return fail(ILL_E_ARG, "q4 quantize: bad shape %lld x %d", (long long)rows, cols);
  illq::parallel_rows(rows, threads, [&](int64_t a, int64_t b) { illq::quant_rows_q4(w, a, b, cols, packed, sb); });
  return ILL_OK;
}

int ill_quantize_q8(const float* w, int64_t rows, int cols, int group, int8_t* codes, uint16_t* scales, int threads) {
  if (!w || !codes || !scales || rows < 1 || (group != 32 && group != 64) || cols < group || cols % group)
    return fail(ILL_E_ARG, "q8 quantize: bad shape %lld x %d or group %d", (long long)rows, cols, group);
  illq::parallel_rows(rows, threads, [&](int64_t a, int64_t b) { illq::quant_rows_q8(w, a, b, cols, group, codes, scales); });
  return ILL_OK;
}

int ill_gemv_info(const ill_gemv* g, int* slices, int* blocks_per_slice, int64_t* bytes_per_copy) {
  if (!g) return fail(ILL_E_ARG, "null gemv");
  if (slices) *slices = g->ks;
  if (blocks_per_slice) *blocks_per_slice = g->bps;
  if (bytes_per_copy) *bytes_per_copy = (int64_t)g->rows * g->K / 2 + (int64_t)g->rows * (g->K / 64) * 4;
  return ILL_OK;
}

// ---- tokenizer (host code; ill_tok.h) -----------------------------------------------------
struct ill_tok {
  iltk::Tok t;
};

namespace {
int tok_ids_out(const std::vector<int32_t>& v, int32_t* ids, int64_t cap, int64_t* n) {
  *n = (int64_t)v.size();
  if ((int64_t)v.size() > cap) return fail(ILL_E_ARG, "%lld ids do not fit a buffer of %lld", (long long)v.size(), (long long)cap);
  if (!v.empty()) memcpy(ids, v.data(), v.size() * 4);
  return ILL_OK;
}
int tok_bytes_out(const std::string& s, char* out, int64_t cap, int64_t* len) {
  *len = (int64_t)s.size();
  if ((int64_t)s.size() > cap) return fail(ILL_E_ARG, "%lld bytes do not fit a buffer of %lld", (long long)s.size(), (long long)cap);
  if (!s.empty()) memcpy(out, s.data(), s.size());
  return ILL_OK;
}
bool tok_text_ok(const char* text, int64_t len) {
  return len == 0 || (text && len > 0 && iltk::utf8_valid((const uint8_t*)text, (size_t)len));
}
}  // namespace

int ill_tok_open(const char* path, ill_tok** out) {
  if (!path || !out) return fail(ILL_E_ARG, "null tokenizer path or handle");
  *out = nullptr;
  ill_tok* t = new ill_tok();
  const std::string err = iltk::open(path, t->t);
  if (!err.empty()) {
    delete t;
    return fail(ILL_E_FILE, "%s", err.c_str());
  }
  *out = t;
  return ILL_OK;
}

int ill_tok_close(ill_tok* t) {
  delete t;
  return ILL_OK;
}

int ill_tok_info(const ill_tok* t, int32_t info[4]) {
  if (!t || !info) return fail(ILL_E_ARG, "null tokenizer");
  info[0] = (int32_t)t->t.n_total;
  info[1] = t->t.im_start;
  info[2] = t->t.im_end;
  info[3] = t->t.eot;
  return ILL_OK;
}

int ill_tok_encode(const ill_tok* t, const char* text, int64_t len, int specials, int32_t* ids, int64_t cap, int64_t* n) {
  if (!t || !n || (cap > 0 && !ids)) return fail(ILL_E_ARG, "bad tokenizer arguments");
  if (!tok_text_ok(text, len)) return fail(ILL_E_ARG, "text is not UTF-8");
  std::vector<int32_t> v;
  iltk::encode(t->t, (const uint8_t*)text, (size_t)len, specials != 0, v);
  return tok_ids_out(v, ids, cap, n);
}

int ill_tok_encode_chat(const ill_tok* t, const char* system, int64_t slen, const char* user, int64_t ulen, int32_t* ids, int64_t cap,
                        int64_t* n) {
  if (!t || !n || (cap > 0 && !ids)) return fail(ILL_E_ARG, "bad tokenizer arguments");
  if (t->t.chat0.empty()) return fail(ILL_E_ARG, "the tokenizer has no <|im_start|> / <|im_end|> tokens");
  if (!tok_text_ok(system, slen) || !tok_text_ok(user, ulen)) return fail(ILL_E_ARG, "text is not UTF-8");
  std::string s = t->t.chat0;
  s.append(system ? system : "", (size_t)slen);
  s += t->t.chat1;
  s.append(user ? user : "", (size_t)ulen);
  s += t->t.chat2;
  std::vector<int32_t> v;
  iltk::encode(t->t, (const uint8_t*)s.data(), s.size(), true, v);
  return tok_ids_out(v, ids, cap, n);
}

int ill_tok_decode(const ill_tok* t, const int32_t* ids, int64_t n, char* out, int64_t cap, int64_t* len) {
  if (!t || !len || n < 0 || (n > 0 && !ids) || (cap > 0 && !out)) return fail(ILL_E_ARG, "bad tokenizer arguments");
  std::string raw;
  for (int64_t i = 0; i < n; i++) {
    const int32_t id = ids[i];
    if (id < 0 || id >= t->t.n_total) continue;
    raw.append((const char*)t->t.tok_bytes + t->t.tok_off[id], t->t.tok_off[id + 1] - t->t.tok_off[id]);
  }
  return tok_bytes_out(iltk::lossy_utf8((const uint8_t*)raw.data(), raw.size()), out, cap, len);
}

int ill_tok_token_bytes(const ill_tok* t, int32_t id, const char** bytes, int64_t* len) {
  if (!t || !bytes || !len) return fail(ILL_E_ARG, "bad tokenizer arguments");
  if (id < 0 || id >= t->t.n_total) {
    *bytes = "";
    *len = 0;
    return ILL_OK;
  }
  *bytes = (const char*)t->t.tok_bytes + t->t.tok_off[id];
  *len = t->t.tok_off[id + 1] - t->t.tok_off[id];
  return ILL_OK;
}

int ill_tok_normalize(const ill_tok* t, const char* text, int64_t len, char* out, int64_t cap, int64_t* olen) {
  if (!t || !olen || (cap > 0 && !out)) return fail(ILL_E_ARG, "bad tokenizer arguments");
  if (!tok_text_ok(text, len)) return fail(ILL_E_ARG, "text is not UTF-8");
  std::string s;
  if (iltk::needs_nfc(t->t, (const uint8_t*)text, (size_t)len)) iltk::nfc(t->t, (const uint8_t*)text, (size_t)len, s);
  else s.assign(text ? text : "", (size_t)len);
  return tok_bytes_out(s, out, cap, olen);
}

int ill_tok_pretokenize(const ill_tok* t, const char* text, int64_t len, int64_t* ends, int64_t cap, int64_t* n) {
  if (!t || !n || (cap > 0 && !ends)) return fail(ILL_E_ARG, "bad tokenizer arguments");
  if (!tok_text_ok(text, len)) return fail(ILL_E_ARG, "text is not UTF-8");
  std::vector<int64_t> v;
  for (size_t i = 0; i < (size_t)len;) {
    i = iltk::piece_end(t->t, (const uint8_t*)text, i, (size_t)len);
    v.push_back((int64_t)i);
  }
  *n = (int64_t)v.size();
  if (*n > cap) return fail(ILL_E_ARG, "%lld pieces do not fit a buffer of %lld", (long long)*n, (long long)cap);
  if (!v.empty()) memcpy(ends, v.data(), v.size() * 8);
  return ILL_OK;
}

int ill_tok_encode_cb(void* user, const char* text, int32_t* ids, int cap) {
  const ill_tok* t = (const ill_tok*)user;
  if (!t || !text || cap < 0 || (cap > 0 && !ids)) return 0;
  const size_t len = strlen(text);
  if (!iltk::utf8_valid((const uint8_t*)text, len)) return 0;
  std::vector<int32_t> v;
  iltk::encode(t->t, (const uint8_t*)text, len, true, v);
  const size_t k = std::min<size_t>(v.size(), (size_t)cap);
  if (k) memcpy(ids, v.data(), k * 4);
  return (int)std::min<size_t>(v.size(), 0x7fffffff);
}

}  // extern "C"
