"""GPU parity of the one-row decode kernel in the read floor's shape (mxa_gemv_wave.hip) against
the CPU oracle, through the C ABI: bit-exact for Q8_0 / Q4_K / Q6_K.

The kernel takes every one-token K-quant / Q8_0 call whose blocks per row nb = K / 256 are in
{4, 8, 16, 32, 56, 64}, one workgroup per CU;
past one pass its waves take up to 64 row sets each. A wave owns 64 / nb rows (one row of 56
blocks at nb = 56, eight lanes idle); the shapes cover each nb it is built for, N that leaves the
last wave or workgroup partial, N so small that some workgroups' waves only stage the
activations, N at the largest one pass holds on a 256-CU MI355X (14 Q4_K waves of 4 rows, 8
Q8_0, 9 Q6_K per CU) and one row past it, several row sets, with x quantized in the kernel and
with Q8_K blocks from the workspace.
"""

import numpy as np
import pytest
import torch

from matricxon_amd import synthetic as S
from matricxon_amd.gemm import q8k_bytes
from oracle import dequant as D

pytestmark = pytest.mark.gpu

TYPES = [D.Q8_0, D.Q4_K, D.Q6_K]
SHAPES = [(1000, 1024), (1500, 2048), (37, 4096), (1, 4096), (4100, 4096), (2000, 8192),
          (700, 16384), (3, 16384), (4096, 14336), (1500, 14336), (5, 14336)]
# the largest N one round holds per type at K = 4096 on 256 CUs, and one more row
ROUND_EDGE = {D.Q4_K: 14336, D.Q8_0: 8192, D.Q6_K: 9216}


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bit_exact(got: np.ndarray, want: np.ndarray) -> None:
    assert got.shape == want.shape
    diff = np.nonzero(bits(got) != bits(want))
    assert diff[0].size == 0, (f"{diff[0].size} outputs differ from the oracle, first at "
                               f"{diff[0][0]},{diff[1][0]}: {got[diff][0]} vs {want[diff][0]}")


def run_both(gpu, oracle, t, n, k, seed):
    w = S.packed_weight(t, n, k, seed=seed)
    x = S.activations(1, k, seed=seed + 1)
    want = oracle.gemm(t, w, x, n, k)
    wd, xd = dev(w), dev(x)
    assert_bit_exact(host(gpu.matmul(t, wd, xd, n, k)), want)  # x quantized in the kernel
    ws = torch.empty(q8k_bytes(1, k), dtype=torch.uint8, device="cuda")
    gpu.quantize_into(xd, ws)
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    assert_bit_exact(host(gpu.matmul_q8k(t, wd, ws, None, out, 1, n, k)), want)  # Q8_K given


@pytest.mark.parametrize("ggml_type", TYPES)
@pytest.mark.parametrize("n,k", SHAPES)
def test_one_row_wave_kernel_matches_oracle(gpu, oracle, ggml_type, n, k) -> None:
    run_both(gpu, oracle, ggml_type, n, k, seed=n + k + ggml_type)


@pytest.mark.parametrize("ggml_type", TYPES)
@pytest.mark.parametrize("extra", [0, 1])
def test_one_row_wave_kernel_round_edge(gpu, oracle, ggml_type, extra) -> None:
    run_both(gpu, oracle, ggml_type, ROUND_EDGE[ggml_type] + extra, 4096, seed=7 + extra)


# More rows than one pass of the CUs' waves holds: several row sets per wave, for every type and
# row length (the Q6_K vocabulary head included).
ROUNDS_CASES = [(D.Q4_K, 28672, 4096), (D.Q8_0, 14336, 4096), (D.Q4_K, 14336, 8192),
                (D.Q4_K, 57344, 4096), (D.Q4_K, 57345, 4096), (D.Q4_K, 14336, 14336),
                (D.Q8_0, 4097, 14336), (D.Q6_K, 14336, 4096), (D.Q6_K, 4096, 14336),
                (D.Q6_K, 8192, 16384), (D.Q6_K, 128256, 4096), (D.Q4_K, 4096, 14336),
                (D.Q6_K, 6144, 14336), (D.Q8_0, 6000, 14336), (D.Q4_K, 20000, 4096)]


@pytest.mark.parametrize("ggml_type,n,k", ROUNDS_CASES)
def test_one_row_wave_kernel_several_rounds(gpu, oracle, ggml_type, n, k) -> None:
    run_both(gpu, oracle, ggml_type, n, k, seed=n + k)


def test_one_row_wave_kernel_repeated_calls_share_nothing(gpu, oracle) -> None:
    """Back-to-back calls on different activations in one stream: nothing of one call's
    activations or counter survives into the next (the counter is reset by every workgroup)."""
    n, k = 4100, 4096
    w = S.packed_weight(D.Q4_K, n, k, seed=3)
    wd = dev(w)
    xs = [S.activations(1, k, seed=s) for s in (10, 11, 12)]
    outs = [gpu.matmul(D.Q4_K, wd, dev(x), n, k) for x in xs]
    for x, y in zip(xs, outs):
        assert_bit_exact(host(y), oracle.gemm(D.Q4_K, w, x, n, k))


def run_rows(gpu, oracle, t, n, k, m, seed):
    w = S.packed_weight(t, n, k, seed=seed)
    x = S.activations(m, k, seed=seed + 1)
    want = oracle.gemm(t, w, x, n, k)
    wd, xd = dev(w), dev(x)
    assert_bit_exact(host(gpu.matmul(t, wd, xd, n, k)), want)  # x quantized in the kernel
    ws = torch.empty(q8k_bytes(m, k), dtype=torch.uint8, device="cuda")
    gpu.quantize_into(xd, ws)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    assert_bit_exact(host(gpu.matmul_q8k(t, wd, ws, None, out, m, n, k)), want)  # Q8_K given


# Two and three activation rows (8-, 16- and 32-block rows; four rows run the matrix-core kernels
# by default and are checked here too): every row's block values from one read of the weight, the
# last wave partial, Q4_K past one pass (row sets), Q6_K and Q8_0 rows.
ROWS_CASES = [(D.Q4_K, 14336, 4096), (D.Q4_K, 1001, 2048), (D.Q6_K, 4100, 4096),
              (D.Q8_0, 3000, 8192), (D.Q4_K, 28672, 4096), (D.Q4_K, 5000, 8192),
              (D.Q6_K, 14336, 4096), (D.Q8_0, 700, 2048)]


@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("ggml_type,n,k", ROWS_CASES)
def test_decode_two_to_four_rows(gpu, oracle, ggml_type, n, k, m) -> None:
    run_rows(gpu, oracle, ggml_type, n, k, m, seed=n + k + m)


@pytest.mark.parametrize("ggml_type,n,k", ROWS_CASES)
def test_decode_four_rows_on_the_decode_kernels(gpu, oracle, ggml_type, n, k) -> None:
    # with the crossover raised to four tokens, four rows take the decode kernels (Q4_K: the
    # floor-shaped kernel; Q6_K and Q8_0: the pipelined one)
    before = gpu.fused_max_tokens
    gpu.set_fused_max_tokens(4)
    try:
        run_rows(gpu, oracle, ggml_type, n, k, 4, seed=n + k + 40)
    finally:
        gpu.set_fused_max_tokens(before)


# IQ4_XS on float activations (one row, weights of 4 MB and more): every IQ4_XS kernel sums in one
# order, so the one-row result equals row 0 of a two-row call (the pipelined kernel) bit for bit
# (the float64 bound of that order is tested with the other decode kernels); shapes past one pass
# (row sets), 56- and 64-block rows, and the 4 MB boundary on either side.
IQ4_CASES = [(14336, 4096), (4096, 14336), (30000, 4096), (2000, 16384), (7710, 1024),
             (7711, 1024), (4096, 4096)]


@pytest.mark.parametrize("n,k", IQ4_CASES)
def test_one_row_iq4_xs_equals_two_row_call(gpu, n, k) -> None:
    w = dev(S.packed_weight(D.IQ4_XS, n, k, seed=n + k))
    x2 = S.activations(2, k, seed=n + 1)
    one = host(gpu.matmul(D.IQ4_XS, w, dev(x2[:1]), n, k))
    two = host(gpu.matmul(D.IQ4_XS, w, dev(x2), n, k))
    assert_bit_exact(one, two[:1])
    f32 = host(gpu.gemv_f32(D.IQ4_XS, w, dev(x2[:1]), n, k))
    assert_bit_exact(f32, one)
