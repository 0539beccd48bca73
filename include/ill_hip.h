/* C ABI of the MI355X decode engine (libillhip.so).
 *
 * Drop-in for the pass API of the reference's Swift `Engine`
 * (Sources/Engine/Engine.swift); the reference's only C ABI is the one-function shim
 * Sources/CShim/include/cshim.h:3-4, which this header extends in the same style: plain
 * C types, an opaque handle, no GPU types in the signatures.
 *
 * Conventions: every function returns 0 on success or a negative error code; the message
 * of the last error on the calling thread is available from ill_last_error(). The caller
 * owns host arrays; the engine owns device memory. An engine is single-threaded and runs
 * on one HIP stream of one GPU.
 */
#ifndef ILL_HIP_H
#define ILL_HIP_H
#include <stdint.h>

/* The library is built with hidden visibility: these entry points are its only exports. */
#ifndef ILL_API
#define ILL_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ill_engine ill_engine;

enum {
  ILL_OK = 0,
  ILL_E_ARG = -1,      /* bad argument (shape, size, state) */
  ILL_E_FILE = -2,     /* model file missing or malformed */
  ILL_E_HIP = -3,      /* HIP runtime error */
  ILL_E_TIMEOUT = -4,  /* a device-side bounded wait expired (the pass was abandoned) */
  ILL_E_FORMAT = -5    /* weight format not supported by this build */
};

/* Thread-local message of the last failure (never NULL). */
ILL_API const char* ill_last_error(void);

/* Engine(modelPath:maxContext:maxPass:maxSteps:) (Engine.swift:71-232): maps the .ill v1
 * file (ModelFile.swift:73-98), repacks the weights into the device tile layout and copies
 * them to HBM once. max_context is rounded up to a multiple of 64. */
ILL_API int ill_create(const char* ill_path, int max_context, int max_pass, int max_steps, ill_engine** out);
ILL_API int ill_destroy(ill_engine* e);

/* Model facts of the loaded file. */
ILL_API int ill_vocab(const ill_engine* e);
ILL_API int ill_layers(const ill_engine* e);
ILL_API int ill_format(const ill_engine* e);   /* 0 f16, 1 q8, 2 q4 */

/* The 16-int device State (Shaders.swift:37-54): pos, n, step, done, maxctx, maxsteps,
 * eos0, eos1, nver, tspec, passes, accepted, tlmh, nodraft, learned, tree.
 * Host writes it before a request (Engine.swift:945-964). */
ILL_API int ill_set_state(ill_engine* e, const int32_t state[16]);
ILL_API int ill_get_state(ill_engine* e, int32_t state[16]);

/* encodePrefill (Engine.swift:588-601): n tokens at positions state.pos.., lm_head on the
 * last row and a greedy commit (the first generated token lands in out_tokens[step] and
 * becomes the next step's input). write_logits keeps that row's fp32 logits. */
ILL_API int ill_prefill(ill_engine* e, const int32_t* toks, int n, int write_logits);

/* encodeDecodeStep (Engine.swift:605-609): one 1-row step on the last committed token. */
ILL_API int ill_decode_step(ill_engine* e, int write_logits);

/* encodeWidePass / encodeSpecPass + k_commit_spec (Engine.swift:567-579, :503-547;
 * Shaders.swift:246-418 without drafting): one pass over `rows` (<= 16) rows.
 * tree != NULL: the 65-int tree [n, depth[16], parent[16], tok[16], anc[16]] with tok[0] =
 * the last committed token; rows attend to the context and their ancestors, the longest
 * path whose drafts equal their parent's argmax is committed and its K/V compacted.
 * tree == NULL: a chain of toks[0..rows-1] = [last token, drafts...]. */
ILL_API int ill_verify_pass(ill_engine* e, int rows, const int32_t* tree, const int32_t* toks, int write_logits);

/* Record `nsteps` decode steps into one hipGraph; ill_launch_graph replays it. Steps after
 * the stop flag early-exit on the device (Shaders.swift:41). The device also sets the stop
 * flag once a following pass of up to 16 rows would not fit in the context, and
 * ill_set_state refuses a live state without that room, so replays never write K/V past
 * max_context. A captured graph is dropped when tracing is switched on or off. */
ILL_API int ill_capture_steps(ill_engine* e, int nsteps);
ILL_API int ill_launch_graph(ill_engine* e);
/* ill_launch_graph with encodeDecodeStep's writeLogits (Engine.swift:605-609) for every
 * recorded step: afterwards ill_read_logits(e, 0, ..) holds the last executed step's logits. */
ILL_API int ill_launch_graph_logits(ill_engine* e, int write_logits);

ILL_API int ill_sync(ill_engine* e);

/* Pinned host array [max_steps] of committed tokens (-1 = not yet written): poll it with
 * volatile loads, as the reference does with ill_volatile_load (cshim.h:4). */
ILL_API const int32_t* ill_out_tokens(ill_engine* e);
ILL_API int ill_reset_out_tokens(ill_engine* e);

/* fp32 logits of pass row `row` from the last pass that wrote logits ([vocab] floats). */
ILL_API int ill_read_logits(ill_engine* e, int row, float* out);

/* Prefix K/V save/load (Engine.swift:788-838) in the reference cache layout:
 * [layer][kv_head][npos][64] f16 bits, for positions 0..npos-1. */
ILL_API int ill_kv_copy_out(ill_engine* e, int npos, uint16_t* k, uint16_t* v);
ILL_API int ill_kv_copy_in(ill_engine* e, int npos, const uint16_t* k, const uint16_t* v);

/* Engine.generate (Engine.swift:922-1038) for one request without drafting: sets the
 * state, prefills `ntok` tokens, then runs decode steps in captured graphs of `chunk`
 * steps while polling out_tokens. Writes up to max_new tokens (stop token excluded) to
 * out and returns their count through n_out; logits_out (optional, [vocab]) receives the
 * first token's logits. */
ILL_API int ill_generate(ill_engine* e, const int32_t* toks, int ntok, int max_new, int chunk,
                 int32_t* out, int* n_out, float* logits_out);

/* Engine.generate's onToken callback (Engine.swift:922, :1024): called on the calling
 * thread with each token as it is delivered; return 0 to stop the request. */
typedef int (*ill_token_fn)(int32_t token, void* user);

/* ill_generate with a per-token callback. When the callback returns 0 the request stops:
 * the steps already queued leave at once (Engine.swift:1032-1036), the K/V cache keeps
 * the prompt and the delivered tokens but the last, and n_out counts the delivered tokens. */
ILL_API int ill_generate_cb(ill_engine* e, const int32_t* toks, int ntok, int max_new, int chunk,
                    int32_t* out, int* n_out, float* logits_out, ill_token_fn on_token, void* user);

/* The host's stop for passes already launched (Engine.swift:1032-1036 writes the State's
 * done flag into shared memory). The word lives in pinned host memory; the commit of every
 * pass reads it (the read is issued when the pass starts): a pass that sees it commits
 * nothing and sets the device State's done flag, so every pass queued behind it leaves at
 * its header. A pass whose commit read the word before the call completes normally.
 * ill_set_state clears it. Safe to call from another thread while a generate call or a
 * launched graph runs. */
ILL_API int ill_stop(ill_engine* e);

/* ---- Speculative decoding with on-device drafting (k_commit_spec, Shaders.swift:246-418) ----
 * With the State's tspec = T > 1, every commit of a prefill or verify pass is speculative: it
 * accepts the longest prefix of the pass's drafts that equals the rows' argmaxes, commits
 * those tokens, then drafts up to T - 1 tokens for the next pass on the device
 * (self-repetition of the output, then the n-gram table, then prompt lookup;
 * Shaders.swift:367-412) and sets up that pass as a chain over [last token, drafts...].
 * The tokens committed equal plain greedy decoding's (every row's logits equal a 1-row
 * step's, bit for bit). The State's passes / accepted fields count passes and accepted
 * drafts (Engine.swift:959). */

/* Engine.loadNGram (Engine.swift:747-753): an n-gram draft table in the NGramTable layout
 * (NGram.swift:1-59): 2^20 slots of {u64 key, i32 next, u16 count, u16 total}, 16 MiB.
 * table NULL (or bytes 0) unloads it. */
ILL_API int ill_load_ngram(ill_engine* e, const void* table, int64_t bytes);

/* The prompt-lookup context of the drafter (promptRecent, Engine.swift:125, :939-942): the
 * last <= 256 of the request's prompt tokens. ill_generate_spec sets it itself. */
ILL_API int ill_set_prompt(ill_engine* e, const int32_t* toks, int n);

/* One verify pass over the rows the last speculative commit drafted (encodeSpecPass /
 * encodeWidePass + k_commit_spec, Engine.swift:524-579), launched and waited for. */
ILL_API int ill_spec_pass(ill_engine* e, int write_logits);

/* Record `npasses` such passes into one hipGraph (Engine.swift:991-1013 encodes them the
 * same way for every format): each pass takes its rows from the commit before it, so the
 * graph chains verify passes without the host; passes after the stop flag early-exit. q4
 * passes run on the pass-kernel instantiation of the State's tspec rows; q8 and f16 passes
 * on the layer-by-layer kernels launched for as many rows, of which the rows a pass does
 * not hold are computed and never committed. ill_launch_graph replays it. */
ILL_API int ill_capture_spec(ill_engine* e, int npasses);

/* Engine.generate with speculation on (Engine.swift:922-1038): prefill, then verify passes
 * of up to `rows` (2..16) rows, in captured graphs of `chunk` passes (every format), while
 * polling out_tokens. adaptive != 0 chooses each pass's
 * shape from the accepted drafts per pass (Engine.nextPassShape, :888-898, with thresholds
 * from this engine's pass costs, which grow with the kernel's row count): the configured
 * shape while at least 2.4 are accepted, 4-row chains while at least 1.6 are (back to the
 * configured shape at 2.2), else one-row passes with a 4-row probe after 16 passes (the
 * gap doubles, up to 128, after each probe that fails). A shape is judged on its own
 * passes, after two of them (one that accepted nothing), with one of them in flight at a
 * time until then; a change to one-row passes cuts the pending drafted pass to its first
 * row. The tokens are those of greedy decoding in every case.
 * out / n_out as for ill_generate; stats (optional, [2]) receives the passes and accepted
 * drafts of the request. */
ILL_API int ill_generate_spec(ill_engine* e, const int32_t* toks, int ntok, int max_new, int rows, int chunk, int adaptive,
                      int32_t* out, int* n_out, int32_t* stats);

/* ---- Learned drafter (ILDraft.swift:1-209, k_ildraft Shaders.swift:421-872) ----------------
 * A table in the ILDRAFT1 format (tools/draft/ildraft.py:16-53) scores the candidates of the
 * n-gram statistics, self-repetition, prompt lookup, the request's TF-IDF neighbours'
 * outputs and the copy candidates with 53 features and a small MLP; a drafting kernel runs
 * it after each speculative commit and proposes the next pass: a chain of up to
 * chain_rows - 1 tokens, or a best-first tree of up to tree_budget tokens (8 children per
 * expansion) verified in one tree pass. Speculation never changes the tokens committed.
 *
 * ill_ildraft_open (ILDraft.init, :38-84): reads and checks a table (NULL on error, see
 * ill_last_error). ill_ildraft_prepare (ILDraft.prepare, :110-208): the per-request context
 * from the user prompt's ids inside the chat template, its text and the tokenizer
 * (`encode` writes the ids of a text into ids[0..cap) and returns their count; NULL: no
 * space-variant candidates). ill_ildraft_request copies the prepared context (the
 * IllDraftReq layout of instantllm_amd/csrc/ill_ildraft.h) and returns its size in bytes. */
typedef struct ill_ildraft ill_ildraft;
typedef int (*ill_encode_fn)(void* user, const char* text, int32_t* ids, int cap);
ILL_API ill_ildraft* ill_ildraft_open(const char* path);
ILL_API void ill_ildraft_close(ill_ildraft* d);
ILL_API int ill_ildraft_prepare(ill_ildraft* d, const int32_t* prompt, int n, const char* text, ill_encode_fn encode, void* user);
ILL_API int64_t ill_ildraft_request(const ill_ildraft* d, void* out, int64_t bytes);

/* Engine.loadLearnedDrafter (Engine.swift:901-904): loads a table into the engine. */
ILL_API int ill_load_ildraft(ill_engine* e, const char* path);

/* Engine.setDraftContext (Engine.swift:908-913): prepares the next ill_generate_spec
 * request's drafter context (at once, on the CPU). That call then drafts with the learned
 * drafter (Engine.swift:950-956) and consumes the context. */
ILL_API int ill_set_draft_context(ill_engine* e, const int32_t* prompt, int n, const char* text, ill_encode_fn encode, void* user);

/* Engine.useLearned / learnedT / learnedTree (Engine.swift:871-880): use != 0 lets a
 * prepared context switch ill_generate_spec to the learned drafter; its passes are chains
 * of chain_rows (2..16) rows, or with tree_budget > 0 trees of min(tree_budget, 15) drafts
 * (passes of that + 1 rows; with ill_generate_spec's `adaptive` these are its configured
 * shape). Defaults 1, 8, 15. */
ILL_API int ill_set_learned(ill_engine* e, int use, int chain_rows, int tree_budget);

/* The pass the last speculative commit set up (no reference counterpart: inspection for
 * tests and tools): info = [mode (1 chain, 2 tree), rows, commit, drafting still pending];
 * toks [16] the rows' tokens; tree [65] the tree buffer (Shaders.swift:23-30 layout). */
ILL_API int ill_pending_pass(ill_engine* e, int32_t info[4], int32_t toks[16], int32_t tree[65]);

/* ---- Prefix reuse across requests (Engine.swift:788-838, :929-933, :1029-1031) ----------
 * ill_generate / ill_generate_spec keep the tokens whose K/V stay valid after the call (the
 * prompt and every generated token but the last); the next call prefills only the part of
 * its prompt after the longest common prefix (at least one token). Any pass or K/V write
 * launched outside those calls forgets the cached tokens.
 * ill_prefix_info: the cached token count and the tokens the last generate call prefilled.
 * ill_save_prefix (Engine.savePrefix): writes the K/V of the first n cached tokens (toks
 * must be that prefix) to `path`: [u64 key: magic, model file size, mtime s, mtime ns,
 * max_context][u64 n][n x i32 tokens][K][V], K and V as [layer][kv head][n][64] f16.
 * ill_load_prefix (Engine.loadPrefix): loads such a file if it was saved for this model
 * file and context (else ILL_E_FILE), makes its tokens the cached prefix and returns them
 * in toks (max_toks entries; NULL to skip) and their count in n_out. */
ILL_API int ill_prefix_info(ill_engine* e, int* cached, int* last_prefill);
/* Engine.truncateCache (Engine.swift:850-853): forget the cached K/V beyond the first n
 * tokens (0 clears the cache). A reused prefix changes where the prompt's last tokens are
 * computed (its K/V come from the earlier request's passes), so a near tie can resolve
 * differently than from a cold cache; callers comparing runs clear it first. */
ILL_API int ill_truncate_cache(ill_engine* e, int n);
ILL_API int ill_save_prefix(ill_engine* e, const char* path, const int32_t* toks, int n);
ILL_API int ill_load_prefix(ill_engine* e, const char* path, int32_t* toks, int max_toks, int* n_out);

/* Timing (Engine.profile / gpuTime, Engine.swift:621-729): GPU milliseconds of `iters`
 * replays of the captured graph, measured with HIP events on the engine's stream. */
ILL_API int ill_time_graph(ill_engine* e, int iters, float* ms);

/* GPU milliseconds of the most recent single pass (prefill chunk, decode step or verify
 * pass launched through the functions above), from HIP events around its kernel. */
ILL_API int ill_last_pass_ms(ill_engine* e, float* ms);

/* Per-workgroup timeline of the pass kernel (the persistent-kernel counterpart of
 * Engine.profile's per-kernel times): when on, thread 0 of every workgroup stores the
 * 100 MHz device clock at points of its role in every layer l (slot 16 l + k: k = 0 role
 * start, 1 input ready, 11 done, 2-10 and 12-15 role-specific intermediate points), and
 * of the lm_head and commit tail (slots 480 + k). Unreached slots stay 0.
 * ill_trace_read copies [256][slots] u64 values of the last pass and returns `slots`. */
ILL_API int ill_trace_enable(ill_engine* e, int on);
ILL_API int ill_trace_read(ill_engine* e, uint64_t* out, int* slots);

/* Stand-alone q4 GEMV, the decode step's matrix-vector product measured on its own
 * The reference has no separate entry for it: it times the same
 * kernels (q4_chunk_norm / q_rows, k_lm_head_T; Shaders.swift:1001-1185, :1327-1364) inside
 * Engine.profile (Engine.swift:639-729). codes [rows][K/2] and scales [rows][K/64] (f16
 * scale | f16 min << 16) are the .ill q4 layout; `copies` device copies of the weights are
 * rotated through so that repeated runs stream from HBM rather than the 256 MB MALL.
 * ill_gemv_run: y = W * rmsnorm(x) * gamma (gamma NULL: y = W * x), `iters` timed runs;
 * y (host [rows], optional) and argmax (host, optional: lowest index of the maximum,
 * which also enables the argmax epilogue) are from the last run. */
typedef struct ill_gemv ill_gemv;
ILL_API int ill_gemv_create(int rows, int K, const uint8_t* codes, const uint32_t* scales, int copies, ill_gemv** out);
ILL_API int ill_gemv_run(ill_gemv* g, const float* x, const float* gamma, int iters, float* y, int32_t* argmax, float* us_per_iter);
ILL_API int ill_gemv_info(const ill_gemv* g, int* slices, int* blocks_per_slice, int64_t* bytes_per_copy);

/* No counterpart in the reference: ill_gemv_run for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). One product on weight copy `copy` of g, enqueued on `stream` (a hipStream_t;
 * NULL: g's own stream) and not waited for. x [K], gamma [K] (NULL: plain input), y [rows]
 * and argmax (one int32) are device pointers owned by the caller; y may be NULL when
 * argmax is not (the product then lives in the library's per-GPU scratch array, at most
 * 262144 rows; larger products need a y buffer). The call allocates nothing: the argmax
 * keys live in that same fixed scratch array, shared by every call on the GPU, so calls
 * that overlap on one GPU race. Same arithmetic and results as ill_gemv_run. */
ILL_API int ill_gemv_run_noalloc(ill_gemv* g, int copy, const float* x, const float* gamma, float* y, int32_t* argmax, void* stream);
ILL_API int ill_gemv_destroy(ill_gemv* g);

/* The converter's quantizers (Converter.quantizeQ4Raw / quantGroup and quantizeQ8,
 * Sources/Engine/Convert.swift:252-370), host code that needs no GPU. w is a row-major
 * float32 [rows][cols] matrix; `threads` CPU threads split the rows (any count gives the
 * same bytes).
 * q4: packed [rows][cols/2] codes (column 2j in the low nibble of byte j) and sb
 * [rows][cols/64][2] f16 bits (scale, bias): per 64 columns the clipped-range search with a
 * least-squares refit that keeps the lowest squared error after f16 rounding.
 * q8: codes [rows][cols] and scales [rows][cols/group] f16 bits, group 32 (the reference) or
 * 64: symmetric, scale = f16(amax/127) raised one ulp when a code would leave -127..127. */
ILL_API int ill_quantize_q4(const float* w, int64_t rows, int cols, uint8_t* packed, uint16_t* sb, int threads);
ILL_API int ill_quantize_q8(const float* w, int64_t rows, int cols, int group, int8_t* codes, uint16_t* scales, int threads);

/* The tokenizer (Sources/Tokenizer: Tokenizer.swift, Core.swift; host code, no GPU):
 * Qwen2 byte-level BPE, equal to Hugging Face `tokenizers` on the same tokenizer.json.
 * `python -m instantllm_amd.tokenizer compile tokenizer.json out.iltk` writes the file
 * (Tokenizer.compile, Compile.swift:14-371) that ill_tok_open maps (Tokenizer(path:),
 * Tokenizer.swift:57-117). ill_tok_info: ids in total (vocabulary and added tokens), and the
 * ids of <|im_start|>, <|im_end|>, <|endoftext|> (-1: absent).
 * ill_tok_encode: `specials` 0 is Tokenizer.encode (:150-152, no added-token matching),
 * 1 is encodeWithSpecials (:154-158, added tokens matched leftmost-longest on the raw text);
 * ill_tok_encode_chat is encodeChat (:160-183, the chat template around system and user);
 * ill_tok_decode is decode (:275-295: the tokens' bytes, ill-formed UTF-8 replaced by U+FFFD,
 * ids without a token skipped); ill_tok_token_bytes is tokenBytes (:266-271, valid while
 * the tokenizer is open); ill_tok_normalize and ill_tok_pretokenize are normalize and
 * preTokenize (:299-323: the NFC text, and the end offsets of the pieces of an NFC text).
 * Text arguments are UTF-8 of the given byte length (anything else: ILL_E_ARG). Output
 * buffers hold `cap` entries; the count or length is always written, and when it exceeds
 * cap the call fails with ILL_E_ARG. ill_tok_encode_cb is an ill_encode_fn over an ill_tok
 * (the `user` argument): encodeWithSpecials of a NUL-terminated text, the first cap ids
 * written and their whole count returned (0 for text that is not UTF-8). */
typedef struct ill_tok ill_tok;
ILL_API int ill_tok_open(const char* path, ill_tok** out);
ILL_API int ill_tok_close(ill_tok* t);
ILL_API int ill_tok_info(const ill_tok* t, int32_t info[4]);
ILL_API int ill_tok_encode(const ill_tok* t, const char* text, int64_t len, int specials, int32_t* ids, int64_t cap, int64_t* n);
ILL_API int ill_tok_encode_chat(const ill_tok* t, const char* system, int64_t slen, const char* user, int64_t ulen, int32_t* ids,
                                int64_t cap, int64_t* n);
ILL_API int ill_tok_decode(const ill_tok* t, const int32_t* ids, int64_t n, char* out, int64_t cap, int64_t* len);
ILL_API int ill_tok_token_bytes(const ill_tok* t, int32_t id, const char** bytes, int64_t* len);
ILL_API int ill_tok_normalize(const ill_tok* t, const char* text, int64_t len, char* out, int64_t cap, int64_t* olen);
ILL_API int ill_tok_pretokenize(const ill_tok* t, const char* text, int64_t len, int64_t* ends, int64_t cap, int64_t* n);
ILL_API int ill_tok_encode_cb(void* user, const char* text, int32_t* ids, int cap);

#ifdef __cplusplus
}
#endif
#endif
