"""The fp32-activation GEMV (`mxa_gemv_f32`, the device counterpart of the reference's Numba
kernels `qgemv_q4_k` / `qgemv_q6_k` / `qgemv_q8_0` / `qgemv_iq4_xs`).

Parity against the Numba kernels themselves is unpinned: numba is not importable here, so they
cannot run. What fixes the result is the mathematics: y = x @ dequant(W).T with x unquantized. The
reference is that product in float64 over the oracle's bit-exact dequantization, and the kernel
must meet it to float32 accuracy: rel-L2 <= 1e-5 and max|diff| <= 1e-4 * max|ref| (ten times
tighter than the north-star bound of 1e-4 / 2e-3, which the Q8_K path meets with room; the Q8_K
path itself misses these bounds by orders of magnitude, which the last tests use to show that this
path really keeps x in float32)."""

import numpy as np
import pytest
import torch

from matricxon_amd import synthetic as S
from matricxon_amd.device_packed import DevicePackedLinear
from matricxon_amd.quantized_gemv import GEMV_KERNELS, qgemv_q4_k
from oracle import dequant as D
from tests.test_gpu_kernels import assert_within_tolerance, dev, host

pytestmark = pytest.mark.gpu

F32_REL_L2 = 1e-5
F32_MAX_REL = 1e-4
TYPES = [D.Q8_0, D.Q4_K, D.Q6_K, D.IQ4_XS]


def product64(t: int, w: np.ndarray, x: np.ndarray, n: int, k: int) -> np.ndarray:
    """(M, N) float64: x @ dequant(W).T."""
    wf = D.dequantize_matrix(t, w, n, k).astype(np.float64)
    return x.astype(np.float64) @ wf.T


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    return float(np.linalg.norm(got.astype(np.float64) - want) / max(np.linalg.norm(want), 1e-30))


def assert_f32_accurate(got: np.ndarray, want: np.ndarray) -> None:
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    rel = rel_l2(got, want)
    mx = np.abs(got.astype(np.float64) - want).max()
    assert rel <= F32_REL_L2, f"rel-L2 {rel:.3e}"
    assert mx <= F32_MAX_REL * np.abs(want).max(), f"max|diff| {mx:.3e}"
    assert_within_tolerance(got, want)  # the north-star bound, a fortiori


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n,k", [(333, 4096), (70, 256), (200, 16640), (96, 14336)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 9])
def test_gemv_f32_matches_float64_product(gpu, t, n, k, m) -> None:
    # (333, 4096): pipelined kernel, rows across workgroups; (70, 256): one block per row, rows
    # 210 / 136 bytes long for Q6_K / IQ4_XS (not 16-byte aligned); (200, 16640): 65 blocks per
    # row, the multi-pass kernel; (96, 14336): 56 blocks, the pipelined kernel at one row and the
    # multi-pass kernel above (the activations outgrow the pipelined kernel's LDS share).
    # m > 4 runs in passes of four rows.
    w = S.packed_weight(t, n, k, seed=7000 + 31 * t + k + n)
    x = S.activations(m, k, seed=7100 + m + k)
    y = host(gpu.gemv_f32(t, dev(w), dev(x), n, k))
    assert_f32_accurate(y, product64(t, w, x, n, k))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("m", [1, 3])
def test_gemv_f32_long_ranges(gpu, t, m) -> None:
    # 30000 rows of 9 blocks: each weight wave's range wraps the block-value ring (rows folded as
    # stages complete); checked on a spread of rows
    n, k = 30000, 2304
    w = S.packed_weight(t, n, k, seed=7600 + t)
    x = S.activations(m, k, seed=7601 + m)
    y = host(gpu.gemv_f32(t, dev(w), dev(x), n, k))
    rows = np.unique(np.concatenate([np.arange(300), np.arange(n - 300, n), np.arange(0, n, 61)]))
    assert_f32_accurate(y[:, rows], product64(t, w[rows], x, len(rows), k))


@pytest.mark.parametrize("t", TYPES)
def test_gemv_f32_one_hot_picks_dequantized_columns(gpu, t) -> None:
    # one-hot rows pick out single weight columns: a wrong element, nibble or sub-block mapping
    # lands on another column's value. The kernel takes d * sc * q - dmin * m with one rounding
    # (an fma) where the dequantizer rounds twice, so equal within a couple of float32 ulps.
    n, k = 130, 512
    w = S.packed_weight(t, n, k, seed=7200 + t)
    cols = [0, 1, 15, 16, 31, 32, 33, 63, 64, 127, 128, 200, 255, 256, 300, 383, 384, 511]
    x = np.zeros((len(cols), k), dtype=np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    y = host(gpu.gemv_f32(t, dev(w), dev(x), n, k))
    want = D.dequantize_matrix(t, w, n, k)[:, cols].T
    tol = 4 * np.finfo(np.float32).eps * np.abs(want) + 1e-30
    assert (np.abs(y.astype(np.float64) - want) <= tol).all()


@pytest.mark.parametrize("t", TYPES)
def test_gemv_f32_keeps_activations_unquantized(gpu, t) -> None:
    # The same call on the Q8_K path is a good deal further from the float64 product than this
    # one: on these inputs the fp32 path's error is orders of magnitude below the Q8_K
    # quantization error (IQ4_XS keeps float activations on both paths).
    n, k = 256, 4096
    w = S.packed_weight(t, n, k, seed=7300 + t)
    x = S.activations(1, k, seed=7301)
    want = product64(t, w, x, n, k)
    e_f32 = rel_l2(host(gpu.gemv_f32(t, dev(w), dev(x), n, k)), want)
    e_q8k = rel_l2(host(gpu.matmul(t, dev(w), dev(x), n, k)), want)
    assert e_f32 <= F32_REL_L2
    if t != D.IQ4_XS:
        assert e_q8k > 100 * e_f32, (e_q8k, e_f32)


@pytest.mark.parametrize("t", [D.Q8_0, D.Q4_K, D.Q6_K])
@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336), (1000, 2048), (30000, 4096),
                                 (5, 16384), (777, 1024)])
def test_gemv_f32_one_row_equals_two_row_call(gpu, t, n, k) -> None:
    # one row takes the floor-shaped kernel (float x staged as [piece][block] with its sums of 16),
    # two rows the pipelined kernel: one summation order, the same bits for the shared row
    w = dev(S.packed_weight(t, n, k, seed=7700 + n + t))
    x2 = S.activations(2, k, seed=7701 + k)
    one = host(gpu.gemv_f32(t, w, dev(x2[:1]), n, k))
    two = host(gpu.gemv_f32(t, w, dev(x2), n, k))
    assert np.array_equal(one.view(np.uint32), two[:1].view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n,k", [(14336, 4096), (8000, 2048), (3000, 8192)])
@pytest.mark.parametrize("m", [2, 3, 4])
def test_float_activation_rows_equal_single_rows(gpu, t, n, k, m) -> None:
    # two to four float-activation rows in one call (the floor-shaped kernel's multi-row forms)
    # give each row the bits of that row alone (IQ4_XS through matmul: it always keeps x float)
    w = dev(S.packed_weight(t, n, k, seed=7800 + n + t + m))
    x = S.activations(m, k, seed=7801 + m)
    call = gpu.matmul if t == D.IQ4_XS else gpu.gemv_f32
    rows = host(call(t, w, dev(x), n, k))
    for r in range(m):
        one = host(call(t, w, dev(x[r:r + 1]), n, k))
        assert np.array_equal(rows[r:r + 1].view(np.uint32), one.view(np.uint32)), f"row {r}"


@pytest.mark.parametrize("n,k,m", [(4096, 4096, 1), (333, 2304, 1), (30000, 512, 1), (700, 4096, 3)])
def test_gemv_f32_iq4_xs_equals_matmul(gpu, n, k, m) -> None:
    # IQ4_XS multiplies float activations on both paths, every kernel in one summation order (one
    # row: the resident kernel where the weight fits it, else the pipelined one): the same bits
    w = S.packed_weight(D.IQ4_XS, n, k, seed=7500 + n + m)
    x = dev(S.activations(m, k, seed=7501 + m))
    wd = dev(w)
    assert torch.equal(gpu.gemv_f32(D.IQ4_XS, wd, x, n, k), gpu.matmul(D.IQ4_XS, wd, x, n, k))


def test_qgemv_mirror_and_registry(gpu) -> None:
    n, k = 300, 4096
    w = S.packed_weight(D.Q4_K, n, k, seed=7400)
    x = S.activations(1, k, seed=7401)
    raw = dev(w).reshape(-1)  # flat bytes, as the reference's memoryview
    y = qgemv_q4_k(dev(x).reshape(k), raw, n, k)
    assert tuple(y.shape) == (n,) and y.dtype == torch.float32
    assert_f32_accurate(host(y)[None, :], product64(D.Q4_K, w, x, n, k))
    for t in TYPES:
        fn, size = GEMV_KERNELS[t]
        wt = S.packed_weight(t, 64, 512, seed=7410 + t)
        assert wt.shape[1] == 512 // D.GEOMETRY[t][0] * size
        xt = S.activations(1, 512, seed=7411)
        yt = fn(dev(xt).reshape(512), dev(wt), 64, 512)
        assert_f32_accurate(host(yt)[None, :], product64(t, wt, xt, 64, 512))
    with pytest.raises(ValueError):
        qgemv_q4_k(dev(x).reshape(k)[:300], raw, n, 300)


@pytest.mark.parametrize("m", [1, 4, 7])
def test_device_packed_linear_numba_backend(gpu, m) -> None:
    # "numba" backend: decode-sized calls on the fp32-activation GEMV, larger ones on a transient
    # dequantization in the layer dtype (float32 here) and a matmul.
    n, k = 512, 4096
    w = S.packed_weight(D.Q6_K, n, k, seed=7500)
    x = S.activations(m, k, seed=7501 + m)
    mod = DevicePackedLinear(dev(w), k, D.Q6_K, dtype=torch.float32, backend="numba")
    y = host(mod(dev(x).reshape(1, m, k))).reshape(m, n)
    assert_f32_accurate(y, product64(D.Q6_K, w, x, n, k))
    native = DevicePackedLinear(dev(w), k, D.Q6_K, dtype=torch.float32, backend="native")
    assert native.backend == "native"
    with pytest.raises(ValueError):
        DevicePackedLinear(dev(w), k, D.Q6_K, backend="cuda")


def test_numba_backend_follows_the_reference_split(gpu) -> None:
    # QuantizedLinear without its native library (quantized_linear.py:94-106): one token takes the
    # GEMV on x cast straight to float32; two rows take the transient dequantization to the layer
    # dtype and `x.to(dtype) @ weight.T`
    n, k = 256, 2048
    w = dev(S.packed_weight(D.Q4_K, n, k, seed=7600))
    mod = DevicePackedLinear(w, k, D.Q4_K, dtype=torch.bfloat16, backend="numba")
    x1 = dev(S.activations(1, k, seed=7601)).reshape(1, 1, k)
    want1 = gpu.gemv_f32(D.Q4_K, w, x1.reshape(1, k), n, k).to(torch.bfloat16).reshape(1, 1, n)
    assert torch.equal(mod(x1), want1)
    x2 = dev(S.activations(2, k, seed=7602)).reshape(1, 2, k)
    weight = gpu.dequantize(w, D.Q4_K).reshape(n, k).to(torch.bfloat16)
    want2 = (x2.reshape(2, k).to(torch.bfloat16) @ weight.T).to(torch.float32).to(torch.bfloat16)
    assert torch.equal(mod(x2), want2.reshape(1, 2, n))
