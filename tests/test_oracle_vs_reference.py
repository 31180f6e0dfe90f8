"""Pins the C restatement of the matmul (oracle/mx_oracle.c) against the reference's own C kernel
`mx_gemm`, compiled from its sources with its flags (oracle/_ref): the results must be equal bit
for bit (the oracle writes the fp32 fold steps as the FMAs gcc forms from the reference's
expressions). Independently of the reference build: on integer activations (lossless Q8_K) the
result must equal the float64 product of the bit-exact dequantized weight up to fp32 rounding of
the per-block folds, and decode rows must equal prefill rows."""

import numpy as np
import pytest

from matricxon_amd import synthetic as S
from oracle import dequant as D

TYPES = [D.Q8_0, D.Q4_K, D.Q6_K, D.IQ4_XS]


@pytest.mark.parametrize("ggml_type", TYPES)
@pytest.mark.parametrize("n_tokens", [1, 3, 9, 16])
def test_oracle_equals_reference_gemm(oracle, ref, ggml_type: int, n_tokens: int) -> None:
    n, k = 33, 1536
    w = S.packed_weight(ggml_type, n, k, seed=ggml_type * 10 + n_tokens)
    x = S.activations(n_tokens, k, seed=n_tokens)
    assert np.array_equal(oracle.gemm(ggml_type, w, x, n, k), ref.gemm(ggml_type, w, x, n, k))


def test_oracle_equals_reference_on_wide_q6_k_scales(oracle, ref) -> None:
    w = S.packed_weight(D.Q6_K, 20, 2048, seed=5, sc_low=-128, sc_high=127)
    x = S.activations(4, 2048, seed=6)
    assert np.array_equal(oracle.gemm(D.Q6_K, w, x, 20, 2048), ref.gemm(D.Q6_K, w, x, 20, 2048))


@pytest.mark.parametrize("ggml_type", TYPES)
def test_exact_on_integer_activations(oracle, ggml_type: int) -> None:
    """The reference's exact check (tests/unit/test_native_gemm.py:95-115)."""
    n, k = 7, 512
    w = S.packed_weight(ggml_type, n, k, seed=ggml_type)
    x = S.integer_activations(3, k, seed=1)
    want = x.astype(np.float64) @ D.dequantize_matrix(ggml_type, w, n, k).astype(np.float64).T
    got = oracle.gemm(ggml_type, w, x, n, k).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-4 * np.abs(want).max())


@pytest.mark.parametrize("ggml_type", TYPES)
def test_close_on_float_activations(oracle, ggml_type: int) -> None:
    """Against float64 of dequant(Q8_K(x)) x dequant(W): what the integer dots compute, exactly,
    before the fp32 folds (IQ4_XS: raw x)."""
    n, k = 16, 1024
    w = S.packed_weight(ggml_type, n, k, seed=100 + ggml_type)
    x = S.activations(2, k, seed=7)
    wd = D.dequantize_matrix(ggml_type, w, n, k).astype(np.float64)
    if ggml_type == D.IQ4_XS:
        xd = x.astype(np.float64)
    else:
        q, d, _ = D.quantize_q8_k(x)
        xd = D.dequantize_q8_k(q, d)
    want = xd @ wd.T
    got = oracle.gemm(ggml_type, w, x, n, k).astype(np.float64)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6


@pytest.mark.parametrize("ggml_type", TYPES)
def test_decode_rows_equal_prefill_rows(oracle, ggml_type: int) -> None:
    n, k = 9, 768
    w = S.packed_weight(ggml_type, n, k, seed=77)
    x = S.activations(6, k, seed=5)
    prefill = oracle.gemm(ggml_type, w, x, n, k)
    for t in range(6):
        assert np.array_equal(oracle.gemm(ggml_type, w, x[t : t + 1], n, k)[0], prefill[t])


def test_supports_only_block_multiples(oracle) -> None:
    assert oracle.supports(D.Q4_K, 3072) and not oracle.supports(D.Q4_K, 3000)
    assert oracle.supports(D.Q8_0, 256) and not oracle.supports(D.Q8_0, 224)
    assert not oracle.supports(10, 3072)  # Q2_K is not one of the four types
