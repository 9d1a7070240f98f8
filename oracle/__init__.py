"""CPU oracle for the W8A8 hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference's (akivet/Mica v0.5/serving) arithmetic for the
three parts of the hot path: the per-token INT8 activation quantizer, the INT8 x INT8 -> INT32 GEMM
with its per-token x per-channel scale epilogue, the RMSNorm it is fused with, the SwiGLU between
the MLP GEMMs and the last-position label readout.  It is the checker the parity tests compare the
HIP kernels against, and the CPU baseline bench.py times.  Nothing in ``mica_amd`` may import it.

Modules
  w8a8      numpy restatement (bf16 as uint16 bit patterns, explicit fp32 steps); every function
            cites the reference file:line it follows.
  gdn       float64 restatement of the GDN token mixer (causal conv + SiLU, l2norm, the gated delta rule
            per token and in chunked WY form, the gated RMSNorm); pinned in tests/test_gdn_oracle.py.
  cpu_path  the reference's own CPU code path (int8_quant.quant_act -> torch._int_mm -> epilogue,
            eager RMSNorm, F.silu) restated with the same torch calls; used as the timed baseline
            and cross-checked bit-for-bit against ``w8a8``.

How each function is pinned (the reference ships no golden vectors for this path) is documented in
the tests: tests/test_oracle.py (known-answer vectors in tests/golden/, closed forms, brute force
on tiny inputs, planted-mistake sensitivity) and tests/native/quotient_check.c.
"""
