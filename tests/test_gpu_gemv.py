"""GPU parity of the stand-alone q4 GEMV (config 1) through the C ABI, against the oracle's
dequantization and RMSNorm in float64: relative L2 <= 1e-2 (the decode-step tolerance)
and the argmax epilogue equal to the lowest-index maximum of the kernel's own outputs.
"""
from __future__ import annotations

import numpy as np
import pytest

from instantllm_amd import synth
from oracle import illread, qwen, metrics

pytestmark = pytest.mark.gpu


def _ref(codes, sb, x, gamma):
    w = illread.dequant_q4(codes, sb).astype(np.float64)
    xx = x.astype(np.float64)
    if gamma is not None:
        xx = qwen.rmsnorm(xx[None, :], gamma.astype(np.float64))[0]
    return w @ xx


@pytest.mark.parametrize("rows,K,norm,amax", [
    (1152, 896, True, False),     # QKV shape
    (896, 4864, False, False),    # down: plain input
    (2048, 896, True, True),      # lm_head-like, argmax epilogue
    (48, 384, True, True),        # small, several slices per tile
])
def test_gemv_matches_oracle(rows, K, norm, amax):
    from instantllm_amd.engine import Gemv
    codes, sb = synth.microbench_q4(1, rows, K)
    x, gamma = synth.microbench_x(1, K)
    x = x[0]
    print(f"gemv {rows}x{K} norm={norm} argmax={amax}", flush=True)
    g = Gemv(codes, np.ascontiguousarray(sb).view(np.uint32).reshape(rows, K // 64), copies=2)
    y, am, us = g.run(x, gamma if norm else None, iters=3, argmax=amax)
    g.close()
    ref = _ref(codes, sb, x, gamma if norm else None)
    assert metrics.rel_l2(y, ref) <= 1e-2
    if amax:
        assert am == int(np.argmax(y))
        assert ref[am] >= ref.max() - 1e-3 * np.abs(ref).max()
