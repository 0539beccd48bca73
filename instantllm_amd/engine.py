"""Python binding of the C ABI (include/ill_hip.h) -- the check/bench harness's view of
the engine. It mirrors the reference's Swift `Engine` API (Sources/Engine/Engine.swift):
`Engine(model_path, max_context, max_pass, max_steps)`, `generate`, the pass encoders
(prefill / decode step / verify pass / commit inside the pass) and the device State.

Everything runs in libillhip.so on the GPU; this module only marshals arguments. There is
no CPU fallback: a missing library raises at import of the engine.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libillhip.so"

ILL_OK, ILL_E_ARG, ILL_E_FILE, ILL_E_HIP, ILL_E_TIMEOUT, ILL_E_FORMAT = 0, -1, -2, -3, -4, -5
TR_DEPTH, TR_PARENT, TR_TOK, TR_ANC, TR_INTS = 1, 17, 33, 49, 65
STATE_FIELDS = ("pos", "n", "step", "done", "maxctx", "maxsteps", "eos0", "eos1",
                "nver", "tspec", "passes", "accepted", "tlmh", "nodraft", "learned", "tree")

_lib = None

# int encode(void* user, const char* text, int32_t* ids, int cap): the tokenizer callback of
# the learned drafter's request context
ENCODE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_char_p, C.POINTER(C.c_int32), C.c_int)
# ill_token_fn: int (*)(int32_t token, void* user)
TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_int32, C.c_void_p)

# The learned drafter's request context as the device reads it (IllDraftReq, ill_ildraft.h)
DRAFT_REQ = np.dtype([("np", "<i4"), ("ncopy", "<i4"), ("nnb", "<i4"), ("nas", "<i4"),
                      ("P", "<i4", 256), ("pprop", "<f4", 256), ("copyTok", "<i4", 256), ("copyInP", "<i4", 256),
                      ("copyPt", "<f4", 256), ("copyF33", "<f4", 256), ("nbScore", "<f4", 16), ("nbOff", "<i4", 17), ("pad", "<i4", 3),
                      ("nbTok", "<i4", 16 * 80), ("asTok", "<i4", 1024), ("asMax", "<f4", 1024), ("asCnt", "<i4", 1024)])


def _encode_cb(encode):
    """(C callback, user pointer) for a tokenizer: an instantllm_amd.tokenizer.Tokenizer (the
    library's own ill_tok_encode_cb on its handle), a function `encode(text: str) ->
    list[int]`, or None (no callback)."""
    if encode is None:
        return ENCODE_FN(), None
    if hasattr(encode, "encode_fn"):
        fn, handle = encode.encode_fn
        return ENCODE_FN(C.cast(fn, C.c_void_p).value), handle

    def cb(_user, text, ids, cap):
        try:
            got = list(encode(text.decode("utf-8")))
        except Exception:
            return 0
        for i, t in enumerate(got[:cap]):
            ids[i] = int(t)
        return len(got)
    return ENCODE_FN(cb), None


class IllError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"ill error {code}: {msg}")
        self.code = code


def load_library(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libillhip.so (built by instantllm_amd/build.py). Raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it with `python instantllm_amd/build.py` "
                           "(the engine has no CPU fallback)")
    lib = C.CDLL(str(p))
    P, I32, F32 = C.c_void_p, C.c_int32, C.c_float
    ip = C.POINTER(C.c_int32)
    sig = {
        "ill_last_error": (C.c_char_p, []),
        "ill_create": (C.c_int, [C.c_char_p, C.c_int, C.c_int, C.c_int, C.POINTER(P)]),
        "ill_destroy": (C.c_int, [P]),
        "ill_vocab": (C.c_int, [P]),
        "ill_layers": (C.c_int, [P]),
        "ill_format": (C.c_int, [P]),
        "ill_set_state": (C.c_int, [P, ip]),
        "ill_get_state": (C.c_int, [P, ip]),
        "ill_prefill": (C.c_int, [P, ip, C.c_int, C.c_int]),
        "ill_decode_step": (C.c_int, [P, C.c_int]),
        "ill_verify_pass": (C.c_int, [P, C.c_int, ip, ip, C.c_int]),
        "ill_capture_steps": (C.c_int, [P, C.c_int]),
        "ill_launch_graph": (C.c_int, [P]),
        "ill_launch_graph_logits": (C.c_int, [P, C.c_int]),
        "ill_sync": (C.c_int, [P]),
        "ill_out_tokens": (ip, [P]),
        "ill_reset_out_tokens": (C.c_int, [P]),
        "ill_read_logits": (C.c_int, [P, C.c_int, C.POINTER(F32)]),
        "ill_kv_copy_out": (C.c_int, [P, C.c_int, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16)]),
        "ill_kv_copy_in": (C.c_int, [P, C.c_int, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16)]),
        "ill_generate": (C.c_int, [P, ip, C.c_int, C.c_int, C.c_int, ip, C.POINTER(C.c_int), C.POINTER(F32)]),
        "ill_generate_cb": (C.c_int, [P, ip, C.c_int, C.c_int, C.c_int, ip, C.POINTER(C.c_int), C.POINTER(F32), TOKEN_FN, P]),
        "ill_stop": (C.c_int, [P]),
        "ill_time_graph": (C.c_int, [P, C.c_int, C.POINTER(F32)]),
        "ill_load_ngram": (C.c_int, [P, C.c_void_p, C.c_int64]),
        "ill_prefix_info": (C.c_int, [P, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
        "ill_save_prefix": (C.c_int, [P, C.c_char_p, ip, C.c_int]),
        "ill_load_prefix": (C.c_int, [P, C.c_char_p, ip, C.c_int, C.POINTER(C.c_int)]),
        "ill_set_prompt": (C.c_int, [P, ip, C.c_int]),
        "ill_truncate_cache": (C.c_int, [P, C.c_int]),
        "ill_spec_pass": (C.c_int, [P, C.c_int]),
        "ill_capture_spec": (C.c_int, [P, C.c_int]),
        "ill_generate_spec": (C.c_int, [P, ip, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, ip, C.POINTER(C.c_int), ip]),
        "ill_last_pass_ms": (C.c_int, [P, C.POINTER(F32)]),
        "ill_trace_enable": (C.c_int, [P, C.c_int]),
        "ill_trace_read": (C.c_int, [P, C.POINTER(C.c_uint64), C.POINTER(C.c_int)]),
        "ill_gemv_create": (C.c_int, [C.c_int, C.c_int, C.POINTER(C.c_uint8), C.POINTER(C.c_uint32), C.c_int, C.POINTER(P)]),
        "ill_gemv_run": (C.c_int, [P, C.POINTER(F32), C.POINTER(F32), C.c_int, C.POINTER(F32), ip, C.POINTER(F32)]),
        "ill_gemv_info": (C.c_int, [P, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int64)]),
        "ill_gemv_destroy": (C.c_int, [P]),
        "ill_gemv_run_noalloc": (C.c_int, [P, C.c_int, P, P, P, P, P]),
        "ill_quantize_q4": (C.c_int, [C.POINTER(F32), C.c_int64, C.c_int, C.POINTER(C.c_uint8), C.POINTER(C.c_uint16), C.c_int]),
        "ill_quantize_q8": (C.c_int, [C.POINTER(F32), C.c_int64, C.c_int, C.c_int, C.POINTER(C.c_int8), C.POINTER(C.c_uint16), C.c_int]),
        "ill_ildraft_open": (P, [C.c_char_p]),
        "ill_ildraft_close": (None, [P]),
        "ill_ildraft_prepare": (C.c_int, [P, ip, C.c_int, C.c_char_p, ENCODE_FN, P]),
        "ill_ildraft_request": (C.c_int64, [P, P, C.c_int64]),
        "ill_load_ildraft": (C.c_int, [P, C.c_char_p]),
        "ill_set_draft_context": (C.c_int, [P, ip, C.c_int, C.c_char_p, ENCODE_FN, P]),
        "ill_set_learned": (C.c_int, [P, C.c_int, C.c_int, C.c_int]),
        "ill_pending_pass": (C.c_int, [P, ip, ip, ip]),
        "ill_tok_open": (C.c_int, [C.c_char_p, C.POINTER(P)]),
        "ill_tok_close": (C.c_int, [P]),
        "ill_tok_info": (C.c_int, [P, ip]),
        "ill_tok_encode": (C.c_int, [P, C.c_char_p, C.c_int64, C.c_int, ip, C.c_int64, C.POINTER(C.c_int64)]),
        "ill_tok_encode_chat": (C.c_int, [P, C.c_char_p, C.c_int64, C.c_char_p, C.c_int64, ip, C.c_int64,
                                          C.POINTER(C.c_int64)]),
        "ill_tok_decode": (C.c_int, [P, ip, C.c_int64, C.c_char_p, C.c_int64, C.POINTER(C.c_int64)]),
        "ill_tok_token_bytes": (C.c_int, [P, C.c_int32, C.POINTER(C.c_char_p), C.POINTER(C.c_int64)]),
        "ill_tok_normalize": (C.c_int, [P, C.c_char_p, C.c_int64, C.c_char_p, C.c_int64, C.POINTER(C.c_int64)]),
        "ill_tok_pretokenize": (C.c_int, [P, C.c_char_p, C.c_int64, C.POINTER(C.c_int64), C.c_int64, C.POINTER(C.c_int64)]),
        "ill_tok_encode_cb": (C.c_int, [P, C.c_char_p, ip, C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _ = I32
    _lib = lib
    return lib


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(C.POINTER(t))


class Engine:
    """One model on one GPU (Engine.swift:71)."""

    def __init__(self, model_path: str, max_context: int = 2048, max_pass: int = 16, max_steps: int = 4096):
        self.lib = load_library()
        h = C.c_void_p()
        self._check(self.lib.ill_create(str(model_path).encode(), max_context, max_pass, max_steps, C.byref(h)))
        self.h = h
        self.vocab = self.lib.ill_vocab(h)
        self.layers = self.lib.ill_layers(h)
        self.format = self.lib.ill_format(h)
        self.max_steps = max_steps
        self.max_context = (max_context + 63) // 64 * 64

    def _check(self, rc: int):
        if rc != ILL_OK:
            raise IllError(rc, self.lib.ill_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self.lib.ill_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- device State (Shaders.swift:37-54) -------------------------------------------
    def set_state(self, pos: int = 0, n: int = 1, maxsteps: int = 64, eos=(151645, 151643), **kw):
        s = dict(pos=pos, n=n, step=0, done=0, maxctx=self.max_context, maxsteps=maxsteps,
                 eos0=eos[0], eos1=eos[1], nver=1, tspec=1)
        s.update(kw)
        a = _i32([s.get(f, 0) for f in STATE_FIELDS])
        self._check(self.lib.ill_set_state(self.h, _ptr(a, C.c_int32)))

    def get_state(self) -> dict:
        a = np.zeros(16, np.int32)
        self._check(self.lib.ill_get_state(self.h, _ptr(a, C.c_int32)))
        return {f: int(v) for f, v in zip(STATE_FIELDS, a)}

    # ---- passes --------------------------------------------------------------------------
    def prefill(self, toks, write_logits: bool = False):
        a = _i32(toks)
        self._check(self.lib.ill_prefill(self.h, _ptr(a, C.c_int32), len(a), int(write_logits)))

    def decode_step(self, write_logits: bool = False):
        self._check(self.lib.ill_decode_step(self.h, int(write_logits)))

    def verify_pass(self, rows: int, tree=None, toks=None, write_logits: bool = False):
        t = _ptr(_i32(tree), C.c_int32) if tree is not None else None
        k = _ptr(_i32(toks), C.c_int32) if toks is not None else None
        self._check(self.lib.ill_verify_pass(self.h, rows, t, k, int(write_logits)))

    def capture_steps(self, n: int):
        self._check(self.lib.ill_capture_steps(self.h, n))

    def launch_graph(self, write_logits: bool = False):
        self._check(self.lib.ill_launch_graph_logits(self.h, int(write_logits)))

    def sync(self):
        self._check(self.lib.ill_sync(self.h))

    def out_tokens(self) -> np.ndarray:
        p = self.lib.ill_out_tokens(self.h)
        return np.ctypeslib.as_array(p, shape=(self.max_steps,))

    def reset_out_tokens(self):
        self._check(self.lib.ill_reset_out_tokens(self.h))

    def read_logits(self, row: int = 0) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        self._check(self.lib.ill_read_logits(self.h, row, _ptr(out, C.c_float)))
        return out

    def kv_copy_out(self, npos: int):
        k = np.empty((self.layers, 2, npos, 64), np.uint16)
        v = np.empty_like(k)
        self._check(self.lib.ill_kv_copy_out(self.h, npos, _ptr(k, C.c_uint16), _ptr(v, C.c_uint16)))
        return k, v

    def kv_copy_in(self, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        npos = k.shape[2]
        self._check(self.lib.ill_kv_copy_in(self.h, npos, _ptr(k, C.c_uint16), _ptr(v, C.c_uint16)))

    def generate(self, tokens, max_new: int, chunk: int = 8, want_logits: bool = False, on_token=None):
        """Engine.generate (Engine.swift:922-1038) without drafting. `on_token(tok) -> bool`
        (optional) sees each token as it is delivered; returning False stops the request."""
        a = _i32(tokens)
        out = np.zeros(max_new, np.int32)
        n = C.c_int(0)
        lg = np.empty(self.vocab, np.float32) if want_logits else None
        lgp = _ptr(lg, C.c_float) if lg is not None else None
        if on_token is None:
            self._check(self.lib.ill_generate(self.h, _ptr(a, C.c_int32), len(a), max_new, chunk,
                                              _ptr(out, C.c_int32), C.byref(n), lgp))
        else:
            cb = TOKEN_FN(lambda t, _user: 1 if on_token(int(t)) else 0)
            self._check(self.lib.ill_generate_cb(self.h, _ptr(a, C.c_int32), len(a), max_new, chunk,
                                                 _ptr(out, C.c_int32), C.byref(n), lgp, cb, None))
        toks = out[: n.value].tolist()
        return (toks, lg) if want_logits else toks

    def stop(self):
        """Stop the passes already launched (Engine.swift:1032-1036): the next commit to read
        the stop word commits nothing and sets the State's done flag."""
        self._check(self.lib.ill_stop(self.h))

    # ---- prefix reuse (Engine.swift:788-838, :929-933) ---------------------------------
    def prefix_info(self) -> tuple[int, int]:
        """(cached tokens, tokens the last generate call prefilled)"""
        c, p = C.c_int(0), C.c_int(0)
        self._check(self.lib.ill_prefix_info(self.h, C.byref(c), C.byref(p)))
        return c.value, p.value

    def save_prefix(self, path: str, tokens):
        a = _i32(tokens)
        self._check(self.lib.ill_save_prefix(self.h, str(path).encode(), _ptr(a, C.c_int32), len(a)))

    def load_prefix(self, path: str) -> list[int]:
        buf = np.zeros(self.max_context, np.int32)
        n = C.c_int(0)
        self._check(self.lib.ill_load_prefix(self.h, str(path).encode(), _ptr(buf, C.c_int32), len(buf), C.byref(n)))
        return buf[: n.value].tolist()

    # ---- speculative decoding (k_commit_spec drafting on the device) ---------------------
    def load_ngram(self, table: np.ndarray | None):
        if table is None:
            self._check(self.lib.ill_load_ngram(self.h, None, 0))
            return
        t = np.ascontiguousarray(table)
        self._check(self.lib.ill_load_ngram(self.h, t.ctypes.data, t.nbytes))

    def truncate_cache(self, n: int = 0):
        """Engine.truncateCache: forget the cached prefix beyond its first n tokens."""
        self._check(self.lib.ill_truncate_cache(self.h, n))

    def set_prompt(self, toks):
        a = _i32(toks)
        self._check(self.lib.ill_set_prompt(self.h, _ptr(a, C.c_int32), len(a)))

    def spec_pass(self, write_logits: bool = False):
        self._check(self.lib.ill_spec_pass(self.h, int(write_logits)))

    def capture_spec(self, npasses: int):
        self._check(self.lib.ill_capture_spec(self.h, npasses))

    def generate_spec(self, tokens, max_new: int, rows: int = 16, chunk: int = 4, adaptive: bool = False):
        """Engine.generate with speculation (Engine.swift:922-1038): (tokens, passes, accepted)."""
        a = _i32(tokens)
        out = np.zeros(max_new, np.int32)
        n = C.c_int(0)
        stats = np.zeros(2, np.int32)
        self._check(self.lib.ill_generate_spec(self.h, _ptr(a, C.c_int32), len(a), max_new, rows, chunk, int(adaptive),
                                               _ptr(out, C.c_int32), C.byref(n), _ptr(stats, C.c_int32)))
        return out[: n.value].tolist(), int(stats[0]), int(stats[1])

    # ---- learned drafter (ILDraft.swift, Engine.swift:865-913) ------------------------------
    def load_ildraft(self, path: str):
        self._check(self.lib.ill_load_ildraft(self.h, str(path).encode()))

    def set_draft_context(self, prompt_ids, text: str, encode=None):
        """Engine.setDraftContext: the next generate_spec call drafts with the learned drafter.
        `encode`: the tokenizer (see _encode_cb)."""
        a = _i32(prompt_ids)
        cb, user = _encode_cb(encode)
        self._check(self.lib.ill_set_draft_context(self.h, _ptr(a, C.c_int32), len(a), text.encode("utf-8"), cb, user))

    def set_learned(self, use: bool = True, chain_rows: int = 8, tree_budget: int = 15):
        self._check(self.lib.ill_set_learned(self.h, int(use), chain_rows, tree_budget))

    def pending_pass(self):
        """(mode, rows, tokens, tree) of the pass the last speculative commit set up."""
        info = np.zeros(4, np.int32)
        toks = np.zeros(16, np.int32)
        tree = np.zeros(TR_INTS, np.int32)
        self._check(self.lib.ill_pending_pass(self.h, _ptr(info, C.c_int32), _ptr(toks, C.c_int32), _ptr(tree, C.c_int32)))
        return int(info[0]), int(info[1]), toks[: info[1]].tolist(), tree

    def last_pass_ms(self) -> float:
        ms = C.c_float(0)
        self._check(self.lib.ill_last_pass_ms(self.h, C.byref(ms)))
        return ms.value

    def trace_enable(self, on: bool = True):
        self._check(self.lib.ill_trace_enable(self.h, int(on)))

    def trace_read(self) -> np.ndarray:
        """[256, slots] device-clock ticks (100 MHz) of the last pass; 0 = not reached."""
        out = np.zeros(256 * 1024, np.uint64)
        n = C.c_int(0)
        self._check(self.lib.ill_trace_read(self.h, _ptr(out, C.c_uint64), C.byref(n)))
        return out[: 256 * n.value].reshape(256, n.value)

    def time_graph(self, iters: int) -> float:
        ms = C.c_float(0)
        self._check(self.lib.ill_time_graph(self.h, iters, C.byref(ms)))
        return ms.value


class Gemv:
    """Stand-alone q4 GEMV (config-1 microbench) over the C ABI: y = W rmsnorm(x) gamma
    (or W x), optional argmax epilogue; `copies` rotated device copies of W."""

    def __init__(self, codes: np.ndarray, scales: np.ndarray, copies: int = 1):
        self.lib = load_library()
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint32)
        self.rows, half = codes.shape
        self.K = 2 * half
        self.h = C.c_void_p()
        rc = self.lib.ill_gemv_create(self.rows, self.K, _ptr(codes, C.c_uint8), _ptr(scales, C.c_uint32), copies,
                                      C.byref(self.h))
        if rc != ILL_OK:
            raise IllError(rc, self.lib.ill_last_error().decode())

    def run(self, x: np.ndarray, gamma: np.ndarray | None = None, iters: int = 1, argmax: bool = False):
        """Returns (y, argmax or None, microseconds per run)."""
        x = np.ascontiguousarray(x, np.float32)
        g = None if gamma is None else np.ascontiguousarray(gamma, np.float32)
        y = np.zeros(self.rows, np.float32)
        am = C.c_int32(-1)
        us = C.c_float(0)
        rc = self.lib.ill_gemv_run(self.h, _ptr(x, C.c_float), None if g is None else _ptr(g, C.c_float), iters,
                                   _ptr(y, C.c_float), C.byref(am) if argmax else None, C.byref(us))
        if rc != ILL_OK:
            raise IllError(rc, self.lib.ill_last_error().decode())
        return y, (int(am.value) if argmax else None), float(us.value)

    def run_noalloc(self, x_dev: int, gamma_dev: int | None, y_dev: int | None, argmax_dev: int | None,
                    copy: int = 0, stream: int | None = None):
        """ill_gemv_run_noalloc: device addresses in, nothing allocated, not waited for."""
        rc = self.lib.ill_gemv_run_noalloc(self.h, copy, x_dev, gamma_dev, y_dev, argmax_dev, stream)
        if rc != ILL_OK:
            raise IllError(rc, self.lib.ill_last_error().decode())

    def info(self) -> dict:
        ks, bps, nbytes = C.c_int(0), C.c_int(0), C.c_int64(0)
        self.lib.ill_gemv_info(self.h, C.byref(ks), C.byref(bps), C.byref(nbytes))
        return {"slices": ks.value, "blocks_per_slice": bps.value, "bytes": int(nbytes.value)}

    def close(self):
        if self.h:
            self.lib.ill_gemv_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)) or 1)


def quantize_q4(w: np.ndarray, threads: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """The converter's q4 quantizer (Convert.swift:286-370) in libillhip.so (CPU code).
    Returns (packed u8 [rows, cols/2], (scale, bias) f16 [rows, cols/64, 2])."""
    lib = load_library()
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    packed = np.empty((rows, cols // 2), np.uint8)
    sb = np.empty((rows, cols // 64, 2), np.uint16)
    rc = lib.ill_quantize_q4(_ptr(w, C.c_float), rows, cols, _ptr(packed, C.c_uint8), _ptr(sb, C.c_uint16),
                             threads or _threads())
    if rc != ILL_OK:
        raise IllError(rc, lib.ill_last_error().decode())
    return packed, sb.view(np.float16)


def quantize_q8(w: np.ndarray, group: int = 32, threads: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """The converter's q8 quantizer (Convert.swift:252-282): (codes i8 [rows, cols],
    scales f16 [rows, cols/group])."""
    lib = load_library()
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    codes = np.empty((rows, cols), np.int8)
    sc = np.empty((rows, cols // group), np.uint16)
    rc = lib.ill_quantize_q8(_ptr(w, C.c_float), rows, cols, group, _ptr(codes, C.c_int8), _ptr(sc, C.c_uint16),
                             threads or _threads())
    if rc != ILL_OK:
        raise IllError(rc, lib.ill_last_error().decode())
    return codes, sc.view(np.float16)


class DraftTable:
    """A learned-drafter table on the host (ILDraft.init / prepare): the per-request context
    the engine would upload, for inspection."""

    def __init__(self, path: str):
        self.lib = load_library()
        h = self.lib.ill_ildraft_open(str(path).encode())
        if not h:
            raise IllError(ILL_E_FILE, self.lib.ill_last_error().decode())
        self.h = h

    def prepare(self, prompt_ids, text: str, encode=None) -> np.ndarray:
        a = _i32(prompt_ids)
        cb, user = _encode_cb(encode)
        rc = self.lib.ill_ildraft_prepare(self.h, _ptr(a, C.c_int32), len(a), text.encode("utf-8"), cb, user)
        if rc != ILL_OK:
            raise IllError(rc, self.lib.ill_last_error().decode())
        n = self.lib.ill_ildraft_request(self.h, None, 0)
        assert n == DRAFT_REQ.itemsize, (n, DRAFT_REQ.itemsize)
        buf = np.zeros(1, DRAFT_REQ)
        self.lib.ill_ildraft_request(self.h, buf.ctypes.data, n)
        return buf[0]

    def close(self):
        if getattr(self, "h", None):
            self.lib.ill_ildraft_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
