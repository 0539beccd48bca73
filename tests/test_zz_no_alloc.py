"""GPU test of the allocation-free GEMV entry point (ill_gemv_run_noalloc) through the C ABI:
its products and argmaxes equal those of ill_gemv_run on the same handle bit for bit, on
two calls in a row (the second with a smaller matrix), with the product kept in the
library's scratch array or in a caller buffer; a product too large for the scratch array
without a caller buffer is refused. Device buffers come from the HIP runtime through
ctypes (hipMalloc / hipMemcpy), outside the entry point under test."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from instantllm_amd import synth

pytestmark = pytest.mark.gpu

SCRATCH_YMAX = 262144


class Hip:
    """The few HIP runtime calls the test needs for its own device buffers."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        self.h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.h.hipFree.argtypes = [C.c_void_p]
        self.h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.h.hipDeviceSynchronize.argtypes = []
        self.bufs = []

    def put(self, a: np.ndarray) -> int:
        p = C.c_void_p()
        assert self.h.hipMalloc(C.byref(p), max(a.nbytes, 4)) == 0
        self.bufs.append(p.value)
        assert self.h.hipMemcpy(p.value, a.ctypes.data, a.nbytes, 1) == 0   # host to device
        return p.value

    def get(self, p: int, like: np.ndarray) -> np.ndarray:
        out = np.empty_like(like)
        assert self.h.hipDeviceSynchronize() == 0
        assert self.h.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0   # device to host
        return out

    def close(self):
        for p in self.bufs:
            self.h.hipFree(p)
        self.bufs = []


def _gemv(rows, K, seed=1, copies=1):
    from instantllm_amd.engine import Gemv
    codes, sb = synth.microbench_q4(seed, rows, K)
    return Gemv(codes, np.ascontiguousarray(sb).view(np.uint32).reshape(rows, K // 64), copies=copies)


def test_noalloc_equals_gemv_run_two_calls():
    hip = Hip()
    try:
        # call 1: 4096 x 896 with the RMSNorm prologue, argmax only (y in the scratch array)
        print("noalloc call 1: 4096 x 896, argmax, y in scratch", flush=True)
        g1 = _gemv(4096, 896, copies=2)
        x, gamma = synth.microbench_x(1, 896)
        x = np.ascontiguousarray(x[0], np.float32)
        y_ref1, am_ref1, _ = g1.run(x, gamma, iters=1, argmax=True)
        dx, dg = hip.put(x), hip.put(gamma)
        dam = hip.put(np.full(1, -7, np.int32))
        g1.run_noalloc(dx, dg, None, dam, copy=1)
        assert int(hip.get(dam, np.zeros(1, np.int32))[0]) == am_ref1
        # the same product into a caller buffer: bit-identical to ill_gemv_run
        dy = hip.put(np.zeros(4096, np.float32))
        g1.run_noalloc(dx, dg, dy, dam, copy=0)
        y1 = hip.get(dy, y_ref1)
        assert np.array_equal(y1.view(np.uint32), y_ref1.view(np.uint32))
        assert int(hip.get(dam, np.zeros(1, np.int32))[0]) == am_ref1
        # call 2: a smaller matrix (1152 x 896, K split over slices), plain input and gamma
        print("noalloc call 2: 1152 x 896, y and argmax", flush=True)
        g2 = _gemv(1152, 896, seed=2)
        x2, _ = synth.microbench_x(2, 896)
        x2 = np.ascontiguousarray(x2[0], np.float32)
        y_ref2, am_ref2, _ = g2.run(x2, None, iters=1, argmax=True)
        dx2 = hip.put(x2)
        dy2 = hip.put(np.zeros(1152, np.float32))
        g2.run_noalloc(dx2, None, dy2, dam)
        y2 = hip.get(dy2, y_ref2)
        assert np.array_equal(y2.view(np.uint32), y_ref2.view(np.uint32))
        assert int(hip.get(dam, np.zeros(1, np.int32))[0]) == am_ref2
        g1.close()
        g2.close()
    finally:
        hip.close()


def test_noalloc_refuses_products_beyond_the_scratch():
    from instantllm_amd.engine import IllError, ILL_E_ARG
    hip = Hip()
    try:
        rows = SCRATCH_YMAX + 16
        print(f"noalloc: {rows} rows without y must be refused", flush=True)
        g = _gemv(rows, 128)
        dx = hip.put(np.ones(128, np.float32))
        dam = hip.put(np.zeros(1, np.int32))
        with pytest.raises(IllError) as ei:
            g.run_noalloc(dx, None, None, dam)
        assert ei.value.code == ILL_E_ARG and "scratch" in str(ei.value)
        with pytest.raises(IllError):
            g.run_noalloc(dx, None, None, None)   # nothing to compute
        with pytest.raises(IllError):
            g.run_noalloc(dx, None, None, dam, copy=1)   # no such weight copy
        g.close()
    finally:
        hip.close()
