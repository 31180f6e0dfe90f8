"""GPU parity of the HIP kernels against the CPU oracle (oracle/), through the C ABI.

Bars (the benchmark's stated tolerances): dequantized values bit-exact; matmul outputs within rel-L2 <= 1e-4 and
max|diff| <= 2e-3 * max|ref| of the reference C kernel semantics. K-quant and Q8_0 outputs are
additionally checked for bit-equality with the oracle: integer block dots are exact and the
kernels fold blocks in the oracle's order with the oracle's fused steps, so any difference there
is a bug, not rounding. IQ4_XS (float activations, a sequential fp32 chain in the reference) is
held to the tolerance only.
"""

import numpy as np
import pytest
import torch

from matricxon_amd import synthetic as S
from oracle import dequant as D

pytestmark = pytest.mark.gpu

TYPES = [D.Q8_0, D.Q4_K, D.Q6_K, D.IQ4_XS]
REL_L2 = 1e-4
MAX_REL = 2e-3


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_within_tolerance(got: np.ndarray, want: np.ndarray) -> None:
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    mx = np.abs(got - want).max()
    assert rel <= REL_L2, f"rel-L2 {rel:.3e}"
    assert mx <= MAX_REL * np.abs(want).max(), f"max|diff| {mx:.3e} vs max|ref| {np.abs(want).max():.3e}"


def check_gemm(gpu, oracle, ggml_type, w, x, n, k, exact=True):
    y = host(gpu.matmul(ggml_type, dev(w), dev(x), n, k))
    want = oracle.gemm(ggml_type, w, x, n, k)
    assert y.shape == want.shape
    assert_within_tolerance(y, want)
    if exact and ggml_type != D.IQ4_XS:
        diff = np.nonzero(bits(y) != bits(want))
        assert diff[0].size == 0, f"{diff[0].size} outputs differ from the oracle, first at {diff[0][0]},{diff[1][0]}"
    return y


# ---------------------------------------------------------------------------- dequantization


def test_half_decoding_all_patterns(gpu) -> None:
    h = np.arange(1 << 16, dtype=np.uint16)
    hf = h.view(np.float16)
    h = h[~np.isinf(hf) & ~np.isnan(hf)]
    blocks = np.zeros((h.size, 34), dtype=np.uint8)
    blocks[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    blocks[:, 2] = 1
    got = host(gpu.dequantize(dev(blocks), D.Q8_0)).reshape(-1, 32)[:, 0]
    assert np.array_equal(bits(got), bits(h.view(np.float16).astype(np.float32)))


@pytest.mark.parametrize("ggml_type", TYPES)
def test_dequantize_bit_exact(gpu, ggml_type) -> None:
    w = S.packed_weight(ggml_type, 96, 2048, seed=300 + ggml_type)
    blocks = w.reshape(-1, D.GEOMETRY[ggml_type][1])
    # force f16-subnormal and zero scales into a few blocks
    off = {D.Q8_0: 0, D.Q4_K: 0, D.Q6_K: 208, D.IQ4_XS: 0}[ggml_type]
    blocks[::7, off : off + 2] = np.frombuffer(np.uint16(0x0003).tobytes(), dtype=np.uint8)
    blocks[1::11, off : off + 2] = 0
    got = host(gpu.dequantize(dev(blocks), ggml_type))
    assert np.array_equal(bits(got), bits(D.dequantize(ggml_type, blocks)))


def test_dequantize_q6_k_wide_scales(gpu) -> None:
    w = S.packed_weight(D.Q6_K, 32, 1024, seed=5, sc_low=-128, sc_high=127)
    got = host(gpu.dequantize(dev(w), D.Q6_K))
    assert np.array_equal(bits(got), bits(D.dequantize(D.Q6_K, w)))


@pytest.mark.parametrize("ggml_type", TYPES)
def test_dequant_rows_gather(gpu, ggml_type) -> None:
    n, k = 50, 1024
    w = S.packed_weight(ggml_type, n, k, seed=17)
    rows = np.array([3, 0, 49, 3, 17, 60, -1], dtype=np.int32)
    got = host(gpu.dequant_rows(ggml_type, dev(w), dev(rows), k))
    full = D.dequantize_matrix(ggml_type, w, n, k)
    for i, r in enumerate(rows):
        if 0 <= r < n:
            assert np.array_equal(bits(got[i]), bits(full[r]))
        else:
            assert np.all(np.isnan(got[i]))


# ---------------------------------------------------------------------------- Q8_K quantizer


@pytest.mark.parametrize("shape", [(1, 256), (3, 4096), (16, 14336), (5, 1024)])
def test_quantize_q8_k_exact(gpu, oracle, shape) -> None:
    x = S.activations(*shape, seed=shape[0] * 7)
    x[0, :256] = 0.0  # an all-zero block
    if shape[1] >= 512:
        x[0, 256:512] = np.linspace(-127, 127, 256, dtype=np.float32) + 0.5  # ties
    q, d, bs = (host(t) for t in gpu.quantize_q8_k(dev(x)))
    wq, wd, wbs = oracle.quantize_q8_k(x)
    assert np.array_equal(q, wq)
    assert np.array_equal(bits(d), bits(wd))
    assert np.array_equal(bs, wbs)


def test_quantize_q8_k_nan_element(gpu, oracle) -> None:
    x = S.activations(1, 256, seed=3)
    x[0, 7] = np.nan
    q, d, _ = (host(t) for t in gpu.quantize_q8_k(dev(x)))
    wq, wd, _ = oracle.quantize_q8_k(x)
    assert np.array_equal(q, wq) and np.array_equal(d, wd)


# ---------------------------------------------------------------------------- matmul

SHAPES = [(7, 512, 1), (7, 512, 3), (16, 1024, 2), (33, 1536, 5), (100, 4096, 16), (1, 256, 1),
          (17, 768, 17), (40, 2048, 33), (129, 14336, 4)]


@pytest.mark.parametrize("ggml_type", TYPES)
@pytest.mark.parametrize("n,k,m", SHAPES)
def test_gemm_matches_oracle(gpu, oracle, ggml_type, n, k, m) -> None:
    w = S.packed_weight(ggml_type, n, k, seed=n * 31 + m)
    x = S.activations(m, k, seed=m * 13 + k)
    check_gemm(gpu, oracle, ggml_type, w, x, n, k)


@pytest.mark.parametrize("ggml_type", TYPES)
def test_gemm_exact_on_integer_activations(gpu, ggml_type) -> None:
    n, k = 7, 512
    w = S.packed_weight(ggml_type, n, k, seed=ggml_type)
    x = S.integer_activations(3, k, seed=1)
    want = x.astype(np.float64) @ D.dequantize_matrix(ggml_type, w, n, k).astype(np.float64).T
    got = host(gpu.matmul(ggml_type, dev(w), dev(x), n, k)).astype(np.float64)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-4 * np.abs(want).max())


def test_gemm_q6_k_wide_scales(gpu, oracle) -> None:
    w = S.packed_weight(D.Q6_K, 48, 2048, seed=5, sc_low=-128, sc_high=127)
    check_gemm(gpu, oracle, D.Q6_K, w, S.activations(6, 2048, seed=6), 48, 2048)


def test_gemm_odd_q6_k_row_alignment(gpu, oracle) -> None:
    """K = 256 x odd: Q6_K rows of 210 x odd bytes start on 2-byte boundaries."""
    w = S.packed_weight(D.Q6_K, 23, 768, seed=9)
    check_gemm(gpu, oracle, D.Q6_K, w, S.activations(3, 768, seed=2), 23, 768)


@pytest.mark.parametrize("ggml_type", TYPES)
def test_decode_rows_equal_prefill_rows(gpu, ggml_type) -> None:
    """tests/unit/test_native_gemm.py:177-189 of the reference, on the GPU: a token's output must
    not depend on whether it was computed alone or in a batch."""
    n, k = 9, 768
    w = dev(S.packed_weight(ggml_type, n, k, seed=77))
    x = S.activations(6, k, seed=5)
    batch = host(gpu.matmul(ggml_type, w, dev(x), n, k))
    for t in range(6):
        alone = host(gpu.matmul(ggml_type, w, dev(x[t : t + 1]), n, k))
        assert np.array_equal(bits(alone[0]), bits(batch[t]))


@pytest.mark.parametrize("m", [17, 64, 512])
def test_iq4_xs_prefill_rows_near_decode_rows(gpu, m) -> None:
    """The one relaxation of tests/unit/test_native_gemm.py:177-189: IQ4_XS batches of 17 rows or
    more run on bf16 matrix cores with x split into hi + lo parts, which sums in another order
    than the decode kernels (and drops x's bits below hi + lo, under 2^-16 of |x|). Each such row
    must stay within the north-star bound of the same token decoded alone: rel-L2 <= 1e-4 and
    max|diff| <= 2e-3 * max|decode row|. Up to 16 rows the equality is bit for bit (above)."""
    n, k = 96, 4096
    w = dev(S.packed_weight(D.IQ4_XS, n, k, seed=78))
    x = S.activations(m, k, seed=500 + m)
    batch = host(gpu.matmul(D.IQ4_XS, w, dev(x), n, k))
    worst = 0.0
    for t in range(m):
        alone = host(gpu.matmul(D.IQ4_XS, w, dev(x[t : t + 1]), n, k))[0]
        assert_within_tolerance(batch[t], alone)
        worst = max(worst, float(np.linalg.norm(batch[t] - alone) / np.linalg.norm(alone)))
    print(f"IQ4_XS M={m}: worst row rel-L2 prefill vs decode {worst:.2e}")


def test_gemm_multi_equals_separate_calls(gpu) -> None:
    k = 1024
    items = [(D.Q4_K, 64), (D.Q4_K, 16), (D.Q6_K, 16)]
    ws = [dev(S.packed_weight(t, o, k, seed=i)) for i, (t, o) in enumerate(items)]
    x = dev(S.activations(3, k, seed=11))
    multi = gpu.matmul_multi([(t, w, o) for (t, o), w in zip(items, ws)], x)
    for (t, o), w, y in zip(items, ws, multi):
        assert torch.equal(y, gpu.matmul(t, w, x, o, k))


# Shared-input weights in one launch (decode, up to 16 tokens): the q/k/v and gate/up shapes of
# the layer config at reduced N, mixed block types, row counts that leave partial workgroups.
MULTI_CASES = [
    ([(D.Q4_K, 512), (D.Q4_K, 128), (D.Q6_K, 128)], 4096, 1),
    ([(D.Q4_K, 700), (D.Q4_K, 700)], 4096, 2),
    ([(D.Q8_0, 96), (D.Q6_K, 33), (D.Q4_K, 65), (D.Q4_K, 1)], 2048, 4),
    ([(D.Q6_K, 300), (D.Q8_0, 40)], 768, 3),
    ([(D.Q4_K, 512), (D.Q4_K, 128), (D.Q6_K, 128)], 4096, 16),
    ([(D.Q4_K, 700), (D.Q4_K, 700)], 4096, 8),
    ([(D.Q8_0, 96), (D.Q6_K, 33), (D.Q4_K, 65), (D.Q4_K, 1)], 2048, 5),
    ([(D.Q6_K, 300), (D.Q8_0, 40)], 768, 11),
    # gate|up shape: 112 rows per workgroup, 7 tiles through 4 LDS tile slots
    ([(D.Q4_K, 14336), (D.Q4_K, 14336)], 4096, 16),
    # q|k|v shape: segments of different types and tile counts
    ([(D.Q4_K, 4096), (D.Q4_K, 1024), (D.Q6_K, 1024)], 4096, 9),
    # one-row and partial-tile segments among larger ones (rows per workgroup by byte share)
    ([(D.Q4_K, 2000), (D.Q6_K, 1), (D.Q4_K, 37)], 4096, 13),
    # one token (the floor-shaped multi-weight kernel): q|k|v and gate|up at full size (gate|up
    # with two row sets per wave), four segments of 8-block rows, 4-block rows, groups past one
    # pass for every type (row sets), mixed types past one pass, and a segment of one workgroup
    ([(D.Q4_K, 4096), (D.Q4_K, 1024), (D.Q6_K, 1024)], 4096, 1),
    ([(D.Q4_K, 14336), (D.Q4_K, 14336)], 4096, 1),
    ([(D.Q8_0, 96), (D.Q6_K, 33), (D.Q4_K, 65), (D.Q4_K, 1)], 2048, 1),
    ([(D.Q8_0, 3000), (D.Q4_K, 5000)], 1024, 1),
    ([(D.Q6_K, 9000), (D.Q4_K, 100)], 4096, 1),
    ([(D.Q6_K, 14336), (D.Q6_K, 14336)], 4096, 1),
    ([(D.Q8_0, 14336), (D.Q8_0, 14335)], 4096, 1),
    ([(D.Q4_K, 28673), (D.Q6_K, 4096), (D.Q8_0, 2048)], 4096, 1),
    ([(D.Q4_K, 8192), (D.Q4_K, 8191)], 8192, 1),
]


@pytest.mark.parametrize("items,k,m", MULTI_CASES)
def test_gemm_multi_single_launch_matches_oracle(gpu, oracle, items, k, m) -> None:
    ws = [S.packed_weight(t, o, k, seed=90 + i) for i, (t, o) in enumerate(items)]
    x_np = S.activations(m, k, seed=91 + m)
    x = dev(x_np)
    multi = gpu.matmul_multi([(t, dev(w), o) for (t, o), w in zip(items, ws)], x)
    for (t, o), w, y in zip(items, ws, multi):
        got = host(y)
        want = oracle.gemm(t, w, x_np, o, k)
        assert np.array_equal(bits(got), bits(want)), f"type {t} ({o} x {k}), {m} tokens"
        assert torch.equal(y, gpu.matmul(t, dev(w), x, o, k))


def test_gemm_multi_into_out_buffer(gpu) -> None:
    k, m = 1024, 1
    items = [(D.Q4_K, 32), (D.Q6_K, 48)]
    ws = [dev(S.packed_weight(t, o, k, seed=i)) for i, (t, o) in enumerate(items)]
    x = dev(S.activations(m, k, seed=3))
    out = torch.empty((m, 80), dtype=torch.float32, device="cuda")
    ys = gpu.matmul_multi([(t, w, o) for (t, o), w in zip(items, ws)], x, out=out)
    assert ys[0].data_ptr() == out.data_ptr()
    assert torch.equal(out[:, 32:], gpu.matmul(D.Q6_K, ws[1], x, 48, k))
    with pytest.raises(ValueError):
        gpu.matmul_multi([(t, w, o) for (t, o), w in zip(items, ws)], x, out=out[:, :40])


def test_unsupported_shapes_fail_loudly(gpu) -> None:
    w = dev(S.packed_weight(D.Q4_K, 4, 512, seed=1))
    x = dev(S.activations(1, 512, seed=1))
    with pytest.raises(RuntimeError, match="status -1"):
        gpu.matmul(10, w, x, 4, 512)  # Q2_K has no kernel here
    with pytest.raises(ValueError):
        gpu.matmul(D.Q4_K, w, x, 5, 512)  # wrong row count
    with pytest.raises(ValueError):
        gpu.matmul(D.Q4_K, w.cpu(), x, 4, 512)  # host tensor


# Shapes for the decode kernel's row/lane geometry (n_tokens <= 4): one wave holds
# R = 64 // blocks-per-row rows, so small K gives many rows per wave and more (row, token) pairs
# than lanes; K > 64 * 256 takes several passes over a row; N not a multiple of the rows per
# workgroup leaves partial tiles and idle waves.
DECODE_SHAPES = [(1, 256, 2), (130, 256, 4), (65, 512, 3), (3, 16640, 1), (5, 16640, 4),
                 (9, 18432, 2), (70, 4096, 4), (29, 2304, 3), (301, 1024, 1)]


@pytest.mark.parametrize("ggml_type", TYPES)
@pytest.mark.parametrize("n,k,m", DECODE_SHAPES)
def test_decode_geometry_matches_oracle(gpu, oracle, ggml_type, n, k, m) -> None:
    w = S.packed_weight(ggml_type, n, k, seed=n * 7 + k + m)
    x = S.activations(m, k, seed=m * 5 + n)
    check_gemm(gpu, oracle, ggml_type, w, x, n, k)


# Shapes for the one-row decode kernel (quad-per-block, whole ranges in LDS): K = 4096 at the
# headline N (four rows per wave, 16 waves) and at small N (fewer waves per workgroup); K = 14336
# and 2304 (groups of a unit cross row ends: 56 and 9 blocks per row); K = 512 (eight rows per
# unit); K = 16640 (more activation groups than waves); Q6_K rows of odd block counts start on
# 2-byte boundaries; N not a multiple of a workgroup's rows leaves idle waves.
ONE_ROW_SHAPES = [(14336, 4096), (1024, 4096), (4096, 14336), (37, 2304), (1000, 512), (9, 768),
                  (5, 16640), (4100, 4096), (1, 256), (300, 1280), (13001, 4096)]


@pytest.mark.parametrize("ggml_type", TYPES)
@pytest.mark.parametrize("n,k", ONE_ROW_SHAPES)
def test_one_row_decode_geometry_matches_oracle(gpu, oracle, ggml_type, n, k) -> None:
    w = S.packed_weight(ggml_type, n, k, seed=n * 3 + k)
    x = S.activations(1, k, seed=n + 11)
    check_gemm(gpu, oracle, ggml_type, w, x, n, k)


@pytest.mark.parametrize("ggml_type", TYPES)
def test_one_row_decode_weight_off_16_byte_boundary(gpu, oracle, ggml_type) -> None:
    """A packed weight that starts 4 bytes past a 16-byte boundary (a slice of a larger buffer):
    every wave's range then starts mid-chunk."""
    n, k = 700, 1024
    w = S.packed_weight(ggml_type, n, k, seed=41)
    buf = torch.zeros(w.size + 4, dtype=torch.uint8, device="cuda")
    buf[4:] = dev(w.reshape(-1))
    wt = buf[4:].view(n, -1)
    x = S.activations(1, k, seed=42)
    y = host(gpu.matmul(ggml_type, wt, dev(x), n, k))
    want = oracle.gemm(ggml_type, w, x, n, k)
    assert_within_tolerance(y, want)
    if ggml_type != D.IQ4_XS:
        assert np.array_equal(bits(y), bits(want))


# Shapes for the batched-decode kernels (4..16 tokens). Rows of up to 16 blocks (a multiple of
# four) go to the per-wave gather kernel: a workgroup owns ceil(N / CUs) rows in tiles of 16, its
# waves two blocks each (one for Q8_0). N = 4100 leaves a one-row tile and a short last workgroup,
# 5000 a four-row tile; the tiles stay resident in LDS up to 8 tiles that fit (14336 x 4096: 56
# rows, a half last tile; Q6_K / Q8_0 at 8192: two tiles; 14000 x 512: one wave, 55 rows); more
# tiles cycle through slots with a barrier-paced fold per tile (20000 x 4096: 5 tiles that do not
# fit, Q6_K with one tile in flight; 30000 x 4096: 8 tiles, a six-row last tile; 40000 x 2048: 10
# tiles of four waves; 50000 x 4096: 13 tiles). Longer rows whose block count is a multiple of
# four take its long form: units of one tile x a part of eight blocks, each with its own staged
# activations, the fold carried from part to part (K = 5120: 20 blocks, a four-block last part;
# 8192: 32; 14336: the down projection's 56, at 1000 rows one tile per workgroup, at 5000 two, so
# a tile's last part hands over to the next tile's first). Other rows take the streaming kernel
# (rows per workgroup max(16, N / CUs)): K = 2304 gives an odd block count, 768 three blocks; 4352
# and 4608 (17 and 18 blocks) stream in parts of 8, Q6_K parts starting on 2-byte boundaries, with
# their sums carried across parts (40000 x 4608: ten tiles of three parts, past the eight-tile
# output ring).
BATCH_SHAPES = [(4100, 4096, 16), (1000, 4096, 8), (300, 8192, 12), (77, 2304, 5), (40, 768, 16),
                (5000, 1024, 16), (23, 768, 7), (260, 5120, 9), (1000, 14336, 16), (50, 4352, 6),
                (14336, 4096, 16), (8192, 4096, 12), (3000, 2304, 13), (14000, 512, 10),
                (20000, 4096, 6), (30000, 4096, 13), (40000, 2048, 5), (50000, 4096, 16),
                (9000, 5120, 12), (40000, 4608, 4), (300, 8192, 16), (5000, 14336, 5),
                # 4-block rows past eight tiles per CU: the gather kernel's ring form with two
                # waves (128 threads, each folding two outputs of a tile)
                (40000, 1024, 11),
                # resident gather form whose last workgroup has 13 rows (one tile of the five the
                # layout holds): its slots and operand staging keep the layout's places
                (20000, 2048, 8)]


@pytest.mark.parametrize("ggml_type", [D.Q8_0, D.Q4_K, D.Q6_K])
@pytest.mark.parametrize("n,k,m", BATCH_SHAPES)
def test_batched_decode_geometry_matches_oracle(gpu, oracle, ggml_type, n, k, m) -> None:
    w = S.packed_weight(ggml_type, n, k, seed=n * 3 + k + m)
    x = S.activations(m, k, seed=m * 11 + n)
    check_gemm(gpu, oracle, ggml_type, w, x, n, k)


# Decode ranges longer than the block-value ring (over 128 blocks per weight wave at 8 waves per
# CU): the form that folds rows as stages complete, with one stage buffer per wave. Block counts
# that do not divide 64 (K = 2304: 9 blocks, 768: 3) put rows across stage and ring boundaries.
LONG_SHAPES = [(30000, 2304, 1), (30000, 2304, 3), (20000, 4096, 2), (90000, 768, 1),
               (17000, 4096, 4)]


@pytest.mark.parametrize("ggml_type", TYPES)
@pytest.mark.parametrize("n,k,m", LONG_SHAPES)
def test_long_range_decode_matches_oracle(gpu, oracle, ggml_type, n, k, m) -> None:
    w = S.packed_weight(ggml_type, n, k, seed=n + k * 7 + m)
    x = S.activations(m, k, seed=m * 17 + k)
    check_gemm(gpu, oracle, ggml_type, w, x, n, k)


# Prefill: 64-row activation tiles of 128 weight rows: N below, at and past whole 128-row tiles, M
# at and past whole 64-row tiles (rows past M repeat row M - 1), odd and long block counts
# (K = 2304: 9 blocks, 14336: 56).
PREFILL_SHAPES = [(129, 768, 128), (260, 2048, 200), (300, 4096, 130), (50, 14336, 140),
                  (513, 2304, 257), (1000, 4096, 320), (300, 2048, 1030), (129, 1024, 1100),
                  (50, 4352, 1024), (513, 2304, 1089),
                  # one block per row, hundreds of workgroups (64- and 128-row activation tiles)
                  (4096, 256, 480), (4096, 256, 800)]


@pytest.mark.parametrize("ggml_type", [D.Q8_0, D.Q4_K, D.Q6_K])
@pytest.mark.parametrize("n,k,m", PREFILL_SHAPES)
def test_prefill_geometry_matches_oracle(gpu, oracle, ggml_type, n, k, m) -> None:
    w = S.packed_weight(ggml_type, n, k, seed=n * 5 + k + m)
    x = S.activations(m, k, seed=m * 7 + n)
    check_gemm(gpu, oracle, ggml_type, w, x, n, k)


# IQ4_XS prefill: one 16-row weight tile per wave, or two where the grid still gives at least two
# rounds of workgroups (N past whole 256-row tiles, M past whole 64-row tiles, one and two blocks)
IQ4_PREFILL_SHAPES = [(4100, 256, 2000), (2048, 512, 4100), (300, 2048, 130), (4100, 256, 1100)]


@pytest.mark.parametrize("n,k,m", IQ4_PREFILL_SHAPES)
def test_iq4_xs_prefill_geometry_within_tolerance(gpu, oracle, n, k, m) -> None:
    w = S.packed_weight(D.IQ4_XS, n, k, seed=n + 3 * k + m)
    x = S.activations(m, k, seed=m + 11)
    y = host(gpu.matmul(D.IQ4_XS, dev(w), dev(x), n, k))
    rows = np.unique(np.concatenate([np.arange(0, n, max(1, n // 200)), np.arange(n - 20, n)]))
    assert_within_tolerance(y[:, rows], oracle.gemm(D.IQ4_XS, w[rows], x, len(rows), k))


@pytest.mark.parametrize("ggml_type", [D.Q8_0, D.Q4_K, D.Q6_K])
@pytest.mark.parametrize("n,k,m", [(130, 256, 4), (5, 16640, 3), (70, 4096, 1), (70, 512, 130)])
def test_decode_on_prequantized_activations(gpu, oracle, ggml_type, n, k, m) -> None:
    """The same kernel reading Q8_K activations from the workspace instead of quantizing them."""
    from matricxon_amd.gemm import q8k_bytes

    w = S.packed_weight(ggml_type, n, k, seed=n + m)
    x = dev(S.activations(m, k, seed=k + m))
    ws = torch.empty(q8k_bytes(m, k), dtype=torch.uint8, device="cuda")
    gpu.quantize_into(x, ws)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    got = host(gpu.matmul_q8k(ggml_type, dev(w), ws, None, out, m, n, k))
    want = oracle.gemm(ggml_type, w, host(x), n, k)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("m", [20, 150, 1030])
def test_gemm_multi_mixed_types_prefill(gpu, oracle, m) -> None:
    """Q8_K-based and IQ4_XS weights sharing one prefill-sized input: the workspace holds both
    the Q8_K activations and the bf16 split of x, and every output equals its separate call."""
    k = 1024
    items = [(D.Q4_K, 48), (D.IQ4_XS, 32), (D.Q6_K, 16)]
    ws = [dev(S.packed_weight(t, o, k, seed=40 + i)) for i, (t, o) in enumerate(items)]
    x_np = S.activations(m, k, seed=12)
    x = dev(x_np)
    multi = gpu.matmul_multi([(t, w, o) for (t, o), w in zip(items, ws)], x)
    for (t, o), w, y in zip(items, ws, multi):
        assert torch.equal(y, gpu.matmul(t, w, x, o, k))
        want = oracle.gemm(t, host(w), x_np, o, k)
        assert_within_tolerance(host(y), want)
