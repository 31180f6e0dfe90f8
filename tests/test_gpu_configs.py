"""Parity at the five benchmark configurations' real shapes, seeded
synthetic inputs as in bench.py. The oracle checks every output where it runs in seconds, and a
spread of rows (first, last, every 97th) of the 128256-row vocab head and of the prefill chunks."""

import numpy as np
import pytest

from matricxon_amd import synthetic as S
from oracle import dequant as D
from tests.test_gpu_kernels import assert_within_tolerance, bits, dev, host

pytestmark = pytest.mark.gpu


def compare(gpu, oracle, t, w, x, n, k, rows=None):
    y = host(gpu.matmul(t, dev(w), dev(x), n, k))
    if rows is None:
        want = oracle.gemm(t, w, x, n, k)
        got = y
    else:
        want = oracle.gemm(t, w[rows], x, len(rows), k)
        got = y[:, rows]
    assert_within_tolerance(got, want)
    if t != D.IQ4_XS:
        assert np.array_equal(bits(got), bits(want))
    return y


def spread(n: int) -> np.ndarray:
    return np.unique(np.concatenate([np.arange(64), np.arange(n - 64, n), np.arange(0, n, 97)]))


def test_config1_q8_0_gemv(gpu, oracle) -> None:
    w = S.packed_weight(D.Q8_0, 4096, 4096, seed=1)
    compare(gpu, oracle, D.Q8_0, w, S.activations(1, 4096, seed=1001), 4096, 4096)


@pytest.fixture(scope="module")
def q4k_14336():
    return S.packed_weight(D.Q4_K, 14336, 4096, seed=2)


@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_config2_q4_k_batched_decode(gpu, oracle, q4k_14336, m) -> None:
    compare(gpu, oracle, D.Q4_K, q4k_14336, S.activations(m, 4096, seed=1002 + m), 14336, 4096)


@pytest.mark.parametrize("m", [1, 16])
def test_config3_q6_k_vocab_head(gpu, oracle, m) -> None:
    n = 128256
    w = S.packed_weight(D.Q6_K, n, 4096, seed=3)
    compare(gpu, oracle, D.Q6_K, w, S.activations(m, 4096, seed=1003 + m), n, 4096, rows=spread(n))


def test_config4_llama3_8b_layer(gpu, oracle) -> None:
    for i, (name, t, n, k) in enumerate(S.LLAMA3_8B_LAYER):
        w = S.packed_weight(t, n, k, seed=40 + i)
        compare(gpu, oracle, t, w, S.activations(16, k, seed=1040 + i), n, k)


@pytest.mark.parametrize("m", [512, 2048])
def test_config5_q4_k_prefill(gpu, oracle, q4k_14336, m) -> None:
    x = S.activations(m, 4096, seed=1005 + m)
    compare(gpu, oracle, D.Q4_K, q4k_14336, x, 14336, 4096, rows=spread(14336)[::4])


@pytest.mark.parametrize("m", [512, 2048])
def test_config5_iq4_xs_prefill(gpu, oracle, m) -> None:
    w = S.packed_weight(D.IQ4_XS, 4096, 4096, seed=5)
    x = S.activations(m, 4096, seed=2005 + m)
    compare(gpu, oracle, D.IQ4_XS, w, x, 4096, 4096, rows=spread(4096)[::2])


@pytest.mark.parametrize("t,m", [(D.Q4_K, 3), (D.IQ4_XS, 4), (D.Q8_0, 2)])
def test_large_weight_decode_rows(gpu, oracle, t, m) -> None:
    """Decode of weights above 64 MB (the ring-buffer streaming kernel, whose LDS slots are reused
    many times per workgroup) at several activation rows, checked on a spread of rows."""
    k = 4096
    n = (72 << 20) // (k // 256 * {D.Q4_K: 144, D.IQ4_XS: 136, D.Q8_0: 272}[t])
    w = S.packed_weight(t, n, k, seed=7)
    compare(gpu, oracle, t, w, S.activations(m, k, seed=2000 + m), n, k, rows=spread(n))
