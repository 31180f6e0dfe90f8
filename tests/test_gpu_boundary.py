"""The reference boundary's remaining knobs on the GPU: the decode / matrix-core crossover
(`mx_set_fused_max_tokens`, app/native/src/mx_gemm.c:11-16), the cached multi-weight plan
(`MultiGemmPlan`, app/native/gemm_multi.py:15-61) and torch-style negative ids in the packed
embedding (`self.packed[ids]`, app/architectures/device_packed.py:81-84)."""

import numpy as np
import pytest
import torch

from matricxon_amd import synthetic as S
from matricxon_amd.device_packed import DevicePackedEmbedding, upload_packed
from matricxon_amd.gemm import HipGemm
from matricxon_amd.gemm_multi import MultiGemmPlan
from oracle import dequant as D
from tests.test_gpu_kernels import assert_within_tolerance, bits, dev, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ggml_type", [D.Q8_0, D.Q4_K, D.Q6_K])
def test_crossover_moves_no_bits(gpu, oracle, ggml_type) -> None:
    """Every crossover setting gives the oracle's bits for 1..4 rows: the decode kernel and the
    matrix-core kernels fold the same block values in the same order."""
    n, k = 200, 2048
    w = S.packed_weight(ggml_type, n, k, seed=31)
    wd = dev(w)
    try:
        for m in (1, 2, 3, 4):
            x = S.activations(m, k, seed=40 + m)
            want = oracle.gemm(ggml_type, w, x, n, k)
            for limit in (0, 1, 3, 4):
                gpu.set_fused_max_tokens(limit)
                assert gpu.fused_max_tokens == limit
                assert (gpu.workspace_bytes(ggml_type, m, k) == 0) == (m <= limit)
                got = host(gpu.matmul(ggml_type, wd, dev(x), n, k))
                assert np.array_equal(bits(got), bits(want)), (m, limit)
    finally:
        gpu.set_fused_max_tokens(3)


@pytest.mark.parametrize("m", [1, 3, 8, 16, 40])
def test_multi_gemm_plan_matches_separate_calls(gpu, oracle, m) -> None:
    """One plan over q|k|v-shaped weights (Q4_K, Q4_K, Q6_K) equals each weight on its own, bit for
    bit (test_shared_projection.py:45-55 in the reference holds the same invariant)."""
    HipGemm.configure("hip")
    k = 1024
    shapes = [(D.Q4_K, 256), (D.Q4_K, 64), (D.Q6_K, 64)]
    ws = [S.packed_weight(t, n, k, seed=50 + i) for i, (t, n) in enumerate(shapes)]
    plan = MultiGemmPlan.build([(t, dev(w), n) for (t, n), w in zip(shapes, ws)], k)
    assert plan is not None and plan.outs == [256, 64, 64]
    x = S.activations(m, k, seed=60 + m)
    ys = plan.run(dev(x))
    assert ys is not None and len(ys) == 3
    for (t, n), w, y in zip(shapes, ws, ys):
        assert y.shape == (m, n)
        assert np.array_equal(bits(host(y)), bits(oracle.gemm(t, w, x, n, k)))


def test_multi_gemm_plan_declines_what_it_cannot_take(gpu) -> None:
    HipGemm.configure("hip")
    w = dev(S.packed_weight(D.Q4_K, 16, 512, seed=1))
    assert MultiGemmPlan.build([(D.Q4_K, w, 16)], 512) is None             # one weight
    assert MultiGemmPlan.build([(D.Q4_K, w, 16), (10, w, 16)], 512) is None  # Q2_K
    assert MultiGemmPlan.build([(D.Q4_K, w, 16), (D.Q4_K, w, 16)], 500) is None
    try:
        HipGemm.configure("numba")  # no library configured: the reference returns None too
        assert MultiGemmPlan.build([(D.Q4_K, w, 16), (D.Q4_K, w, 16)], 512) is None
    finally:
        HipGemm.configure("hip")


def test_embedding_negative_ids_wrap(gpu) -> None:
    vocab, dim = 100, 256
    w = S.packed_weight(D.Q6_K, vocab, dim, seed=9)
    emb = DevicePackedEmbedding(upload_packed(w, vocab, torch.device("cuda")), dim, D.Q6_K,
                                torch.float32)
    full = D.dequantize_matrix(D.Q6_K, w, vocab, dim)
    ids = torch.tensor([-1, 0, -100, 99, 5, -37]).cuda()
    got = host(emb(ids))
    want = full[[99, 0, 0, 99, 5, 63]]
    assert np.array_equal(bits(got), bits(want))
    # outside [-vocab, vocab): a NaN row, never a read outside the table
    bad = host(emb(torch.tensor([vocab, -vocab - 1, 3, 1 << 40]).cuda()))
    assert np.isnan(bad[0]).all() and np.isnan(bad[1]).all() and np.isnan(bad[3]).all()
    assert np.array_equal(bits(bad[2]), bits(full[3]))


def test_multi_gemm_plan_with_iq4_weight(gpu, oracle) -> None:
    """A group with an IQ4_XS weight (float activations) beside K-quants: both workspace parts."""
    HipGemm.configure("hip")
    k, m = 512, 20
    items = [(D.Q4_K, 64), (D.IQ4_XS, 32)]
    ws = [S.packed_weight(t, n, k, seed=70 + i) for i, (t, n) in enumerate(items)]
    plan = MultiGemmPlan.build([(t, dev(w), n) for (t, n), w in zip(items, ws)], k)
    x = S.activations(m, k, seed=5)
    ys = plan.run(dev(x))
    assert np.array_equal(bits(host(ys[0])), bits(oracle.gemm(D.Q4_K, ws[0], x, 64, k)))
    assert_within_tolerance(host(ys[1]), oracle.gemm(D.IQ4_XS, ws[1], x, 32, k))
