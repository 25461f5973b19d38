"""CPU oracle for the shared-mask N:M sparse GEMV — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker (or the timed CPU
baseline). Nothing in `spmv_decode_amd/` imports it; the product path fails
loudly when its HIP library is missing instead of falling back to this code.

Contents and what pins each function (tests/test_oracle.py):

* `nm_oracle.gather_activations`, `gemv_f64`, `gemv_fp32_dense`: the GEMV
  value (triton_spmv.py:56-115, 149-214; microbench_triton_torchmv.py:383-386).
  Pinned by closed forms: one-hot activations reproduce a packed row exactly,
  a one-hot at a pruned position gives zero, linearity under powers of two,
  group-permutation invariance, and brute force over every 2:4 pattern.
* `nm_oracle.spmm_f64`: the batch > 1 extension, row by row. Pinned against
  a float64 dense matmul on the scattered weight and against gemv_f64 row by
  row.
* `nm_oracle.rms_norm_f64`, `rope_f64`, `silu_f64`, `qkv_decode_f64`: the
  decode-layer operations fused around the GEMV (model.py:258-270, 310-322,
  255-256, 182-187). Pinned against torch's float64 library routines
  (F.rms_norm, complex multiplication, F.silu) and closed forms (constant
  input, identity at angle 0, pair norms preserved, quarter turn).
* `nm_oracle.scatter` / `pack`: compressed <-> dense masked weight
  (microbench_triton_torchmv.py:145-164). Pinned by the round trips
  pack(scatter(x)) == x and scatter(pack(W*mask)) == W*mask, bit-exact.
* `nm_oracle.make_sparse`: synthetic packing / index generation
  (src/spmv/nmsparse_linear.py:14-33). Pinned bit-exactly by the golden
  fixtures in tests/golden/, written by importing the reference.
* `nm_oracle.error_metrics`: max_abs, mean_abs, rmse, rel_l2
  (microbench_triton_torchmv.py:408-423). Pinned against hand-computed values.
* `nm_oracle.expected_exception`: the reference wrapper's argument checks
  (triton_spmv.py:245-294). Pinned against tests/golden/wrapper_validation.json:
  the exception type and message the reference wrapper itself raised for 35
  calls (each check failing alone, valid calls, and pairs of faults that fix
  the order), written by tests/golden/make_validation_golden.py with the
  reference imported in the development container (CPU tensors reporting
  is_cuda, the Triton launch stubbed).
* `c_oracle` (ctypes binding of oracle/nm_gemv_ref.c): the same GEMV in plain
  C with fp32 FMA in the reference's in-program order and software
  fp16/bf16 conversions. Pinned by exhaustive conversion checks against
  numpy and by agreement with the fp64 oracle.
"""
