"""CPU oracle of the kernels-community-rs hot paths -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the algorithms the reference implements on the
GPU (each function cites the reference file:line it follows). It exists to
check the HIP kernels: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only as the checker or as
the timed CPU baseline. No product code path calls into it; the product fails
loudly when libkcr_hip.so is missing.

Modules
  numerics   -- bf16 / f16 rounding (round to nearest even) in numpy
  activation -- activation-rs gated and element-wise activations
  rmsnorm    -- rmsnorm forward / backward / weight-gradient reduction
  attention  -- FlashAttention-2 forward (dense, varlen) and backward

Pinning (what checks each function beyond restating its formula) is listed in
each module's docstring and exercised by tests/test_oracle_*.py. The reference
itself is Rust compiled by cuda-oxide for NVIDIA GPUs; it cannot be built or run
in this environment, so there is no oracle/_ref build.
"""
