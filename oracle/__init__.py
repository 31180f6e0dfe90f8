"""CPU oracle for the quantized-native matmul path. TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import, call
or link anything in this package, and only as the checker. The product path (`matricxon_amd`)
never routes through it: when the HIP library is missing, the product fails loudly.

Contents:
* `dequant.py`  numpy float32 restatement of the reference's bit-exact dequantizers
  (Q8_0, Q4_K, Q6_K, IQ4_XS) and of the Q8_K activation quantizer.
* `fused.py`    numpy restatement of the fused producer ops (RMSNorm, silu * up) whose results
  feed the projections.
* `mx_oracle.c` plain-C restatement of the reference `mx_gemm` semantics (Q8_K activations,
  integer block dots, per-block fp32 folds; fp32 dot for IQ4_XS), built by `Makefile` into
  `oracle/_build/libmx_oracle.so`.
* `native.py`   ctypes wrappers over that library and over `oracle/_ref/libmx_ref*.so`, the
  reference's own C sources compiled by `Makefile` (only where `/root/reference` exists; the
  built files travel with the tree).

How each function is pinned (what a plausible mistake would fail):
* dequant_*       the reference C compiled from its own sources (`mx_dequant_rows` for Q4_K
                  with contraction off: bit-exact; IQ4_XS through `mx_gemm` on one-hot
                  activations: bit-exact; Q6_K through `mx_dequant_rows`: 1-ulp-close), the
                  reference's one-block Q8_0 known answer (d=0.5, qs=-16..15), exact f16
                  subnormal decoding, and special cases (d=0, q=0, u=32).
* quantize_q8_k   brute force on tiny inputs (ties at .5, amax=0, the clamp) and the reference C
                  `mx_gemm` on integer activations (lossless Q8_K); the C oracle's quantizer is
                  compared element-wise with this one.
* mx_oracle gemm  the reference C `mx_gemm` (same results up to fp32 fold rounding), and
                  float64 products of the dequantized weights on integer activations.
* rms_norm        the reference C `mx_rms_norm` (a few ulps: its SIMD sum has no fixed order),
                  closed forms (a constant row c gives c / sqrt(c^2 + eps) * w; a zero row gives
                  0; scaling x by 2^k leaves it unchanged when eps is 0).
* silu_mul        the reference C `mx_silu_mul` (a few ulps: expf), silu(0) = 0, and the limits
                  silu(g) -> g for large g, -> 0 for very negative g.
"""
