"""CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import
this package, and only as the checker or the timed CPU baseline. The engine never calls
it: the product path is the HIP library and fails loudly when that is missing.

Contents (each function cites the reference lines it restates):

* `illread`  -- independent reader of the `.ill` v1 file: dequantized fp32 weights in
  the HF [out, in] layout, undoing the kernel row orders.
* `qwen`     -- numpy fp32 forward / KV cache / greedy decoding
  (`tools/reference/qwen_ref.py:75-220`).
* `tree`     -- tree-verify semantics: ancestor attention via sequential path decoding,
  the accept walk and the KV compaction (`Sources/Engine/Shaders.swift:246-418`).
* `metrics`  -- the comparison measures (`tools/reference/compare.py:48-110`,
  `tools/reference/refcommon.py:85-94`).

Pinning: `tests/test_oracle.py` checks `qwen` against golden vectors written by the
reference's own `qwen_ref.py` (script and fixtures under `tests/golden/`), against a
float64 loop-level brute force on tiny inputs, and against invariants (KV-cache decode
== full re-prefill, argmax ties -> lowest id). `illread` is pinned by closed forms on
hand-built tensors.
"""
