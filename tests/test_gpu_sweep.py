"""A fixed-seed random sample of legal shapes through the C ABI against the oracle.

The hand-picked shapes of the other GPU tests follow the kernels' known boundaries; this sample
draws (type, N, K, M) and shared-input groups, bfloat16 calls and grouped MoE routings from wide
ranges, so that geometry no one thought of is exercised too (it found a short last workgroup and a
two-wave ring form that left outputs unwritten). Each case is its own test, so a failure names the
drawn shape. Bars as in test_gpu_kernels.py: K-quants and Q8_0 bit-exact with the oracle, IQ4_XS
within the north-star tolerance; bfloat16 results equal the float32 entry point's result rounded
by torch's cast."""

import numpy as np
import pytest
import torch

from matricxon_amd import synthetic as S
from oracle import dequant as D
from tests.test_gpu_kernels import assert_within_tolerance, bits, dev, host

pytestmark = pytest.mark.gpu

TYPES = [D.Q4_K, D.Q6_K, D.Q8_0, D.IQ4_XS]
BLOCKS = [1, 2, 3, 4, 5, 8, 9, 12, 16, 17, 20, 28, 56]
MAX_WEIGHT_BYTES = 60e6


def draw_matmul(i: int) -> tuple[int, int, int, int]:
    rng = np.random.default_rng(1000 + i)
    t = int(rng.choice(TYPES))
    k = 256 * int(rng.choice(BLOCKS))
    m = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 11, 13, 16, 17, 24]))
    n = int(rng.choice([1, 7, 16, 33, 255, 1000, 4096, 5000, 12000, 20000, 33000, 40000]))
    n = max(1, min(n, int(MAX_WEIGHT_BYTES / (k * 1.07))))
    return t, n, k, m


def draw_group(i: int) -> tuple[list[tuple[int, int]], int, int, bool]:
    rng = np.random.default_rng(2000 + i)
    k = 256 * int(rng.choice(BLOCKS))
    m = int(rng.choice([1, 2, 3, 4, 8, 11, 16, 17, 33]))
    items = [(int(rng.choice(TYPES)), int(rng.choice([1, 16, 33, 128, 1000, 4096])))
             for _ in range(int(rng.integers(1, 5)))]
    return items, k, m, bool(rng.integers(0, 2))


def draw_moe(i: int) -> tuple[int, int, int, list[int]]:
    rng = np.random.default_rng(3000 + i)
    t = int(rng.choice(TYPES))
    k = 256 * int(rng.choice([1, 2, 4, 8, 16, 28, 56]))
    n = int(rng.choice([16, 96, 300, 512, 1408]))
    counts = [int(rng.choice([0, 0, 1, 2, 3, 7, 16, 17, 40])) for _ in range(int(rng.integers(1, 9)))]
    if sum(counts) == 0:
        counts[0] = 1
    return t, n, k, counts


def sampled_rows(n: int) -> np.ndarray:
    return np.unique(np.concatenate([np.arange(0, n, max(1, n // 300)), np.arange(max(0, n - 40), n)]))


def compare(t: int, got: np.ndarray, want: np.ndarray, what: str) -> None:
    assert_within_tolerance(got, want)
    if t != D.IQ4_XS:
        diff = np.nonzero(bits(got) != bits(want))
        assert diff[0].size == 0, f"{what}: {diff[0].size} outputs differ, first at {diff[0][0]},{diff[1][0]}"


@pytest.mark.parametrize("i", range(48))
def test_sampled_matmul_matches_oracle(gpu, oracle, i) -> None:
    t, n, k, m = draw_matmul(i)
    w = S.packed_weight(t, n, k, seed=5000 + i)
    x = S.activations(m, k, seed=6000 + i)
    y = host(gpu.matmul(t, dev(w), dev(x), n, k))
    rows = sampled_rows(n)
    compare(t, y[:, rows], oracle.gemm(t, w[rows], x, len(rows), k), f"type {t} {n}x{k} M={m}")


@pytest.mark.parametrize("i", range(16))
def test_sampled_group_matches_oracle(gpu, oracle, i) -> None:
    items, k, m, bf16 = draw_group(i)
    ws = [S.packed_weight(t, o, k, seed=7000 + 10 * i + j) for j, (t, o) in enumerate(items)]
    xt = dev(S.activations(m, k, seed=8000 + i))
    if bf16:
        xt = xt.to(torch.bfloat16)
    outs = gpu.matmul_multi([(t, dev(w), o) for (t, o), w in zip(items, ws)], xt, bf16=bf16)
    x32 = xt.to(torch.float32)
    x = host(x32)
    for (t, o), w, y in zip(items, ws, outs):
        if bf16:  # the float32 entry point's result on the widened x, rounded by torch
            y32 = gpu.matmul(t, dev(w), x32, o, k)
            assert torch.equal(y.cpu().view(torch.int16), y32.to(torch.bfloat16).cpu().view(torch.int16))
            y = y32
        rows = sampled_rows(o)
        compare(t, host(y)[:, rows], oracle.gemm(t, w[rows], x, len(rows), k), f"group type {t} rows {o}")


@pytest.mark.parametrize("i", range(16))
def test_sampled_grouped_moe_matches_oracle(gpu, oracle, i) -> None:
    t, n, k, counts = draw_moe(i)
    w = np.stack([S.packed_weight(t, n, k, seed=9000 + 10 * i + e) for e in range(len(counts))])
    x = S.activations(sum(counts), k, seed=9500 + i)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    got = host(gpu.matmul_moe(t, dev(w), dev(x), dev(off), max(counts), n, k))
    want = np.zeros_like(got)
    for e, c in enumerate(counts):
        if c:
            want[off[e]:off[e + 1]] = oracle.gemm(t, w[e], x[off[e]:off[e + 1]], n, k)
    compare(t, got, want, f"moe type {t} {n}x{k} counts {counts}")
