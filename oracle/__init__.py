"""CPU oracle for the quant-inference kernel path — TEST INFRASTRUCTURE ONLY.

These modules restate, on the CPU, the reference's own correctness oracles
(baladithyab/cuda-oxide-bench, analysis/wave15-attention-architecture/
reference/ and the harnesses' inline checks); each function cites the
reference file:line it follows.  They are the checker, never the thing
measured or shipped: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this package.  The product path
(cuda-oxide-bench_amd/) never imports it and has no CPU fallback.

Pinning (what makes the oracle trustworthy, tested in tests/test_oracle_*.py):
  gemm  — known-answer tests from oxide-gemm-sol/bench/cublas_correctness_test.py:8-11,
          the closed-form (i%7)*0.01 x (i%11)*0.01 cell value logged at
          cuda-matmul-tc-bf16/ANALYSIS.md:17, fp64 brute force.
  fp8   — e4m3 codec checked against torch.float8_e4m3fn on every code and
          random values; bit-exact KAT with 1/16-multiples (mojo-matmul-fp8/ANALYSIS.md:91-112);
          scale-linearity invariants.
  gqa   — naive vs torch SDPA (as pytorch_reference.py:127-136 does), MHA/MQA
          reductions, shift invariance, causal row 0, V=1, fp64 loops.
  mla   — reduction to the GQA oracle with one KV head, T=1 and identical-token
          special cases, split/merge (log-sum-exp) invariant.
  gdn   — fused vs canonical (I - beta k k^T) form (pytorch_reference_gdn.py:201-213),
          beta=0, delta-rule write (k^T S' = v when beta|k|^2 = 1), alpha=1/beta=0
          read-out, head-grouping equivalence, fp64 loops.
"""
