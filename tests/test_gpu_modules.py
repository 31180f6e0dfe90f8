"""The drop-in modules (DevicePackedLinear / DevicePackedEmbedding, the reference's
app/architectures/device_packed.py interface) on the GPU."""

import numpy as np
import pytest
import torch

from matricxon_amd import synthetic as S
from matricxon_amd.device_packed import (
    DevicePackedEmbedding,
    DevicePackedLinear,
    HipDequantizer,
    upload_packed,
)
from oracle import dequant as D
from tests.test_gpu_kernels import assert_within_tolerance, bits, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ggml_type", [D.Q8_0, D.Q4_K, D.Q6_K, D.IQ4_XS])
def test_linear_forward_matches_oracle(gpu, oracle, ggml_type) -> None:
    n, k = 48, 1024
    w = S.packed_weight(ggml_type, n, k, seed=12)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(1))
    mod = DevicePackedLinear(upload_packed(w, n, torch.device("cuda")), k, ggml_type, bias=bias,
                             dtype=torch.float32)
    x = S.activations(6, k, seed=3).reshape(2, 3, k)
    y = mod(torch.from_numpy(x).cuda())
    assert y.shape == (2, 3, n) and y.dtype == torch.float32
    want = oracle.gemm(ggml_type, w, x.reshape(6, k), n, k) + bias.numpy()
    assert_within_tolerance(host(y).reshape(6, n), want)
    assert mod.out_features == n and mod.in_features == k
    assert "packed" not in mod.state_dict()  # non-persistent, as the reference's buffer


def test_linear_bf16_layer_dtype(gpu, oracle) -> None:
    """In a bf16 model the layer casts x to bf16 first and returns bf16 (device_packed.py:54)."""
    n, k = 32, 512
    w = S.packed_weight(D.Q4_K, n, k, seed=4)
    mod = DevicePackedLinear(upload_packed(w, n, torch.device("cuda")), k, D.Q4_K)
    x = torch.from_numpy(S.activations(1, k, seed=2)).reshape(1, 1, k).cuda()
    y = mod(x)
    assert y.dtype == torch.bfloat16 and y.shape == (1, 1, n)
    xb = x.to(torch.bfloat16).float().cpu().numpy().reshape(1, k)
    want = oracle.gemm(D.Q4_K, w, xb, n, k)
    assert np.array_equal(host(y.float()).reshape(1, n),
                          torch.from_numpy(want).to(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("ggml_type", [D.Q4_K, D.Q6_K])
def test_embedding_lookup_and_tied_head(gpu, oracle, ggml_type) -> None:
    vocab, dim = 300, 512
    w = S.packed_weight(ggml_type, vocab, dim, seed=21)
    emb = DevicePackedEmbedding(upload_packed(w, vocab, torch.device("cuda")), dim, ggml_type,
                                torch.float32)
    ids = torch.tensor([[1, 299, 7], [7, 0, 150]]).cuda()
    got = host(emb(ids))
    full = D.dequantize_matrix(ggml_type, w, vocab, dim)
    assert np.array_equal(bits(got), bits(full[ids.cpu().numpy()]))
    head = emb.as_linear()
    assert head.packed.data_ptr() == emb.packed.data_ptr()  # same bytes, no second copy
    x = S.activations(2, dim, seed=8)
    assert_within_tolerance(host(head(torch.from_numpy(x).cuda())),
                            oracle.gemm(ggml_type, w, x, vocab, dim))


def test_hip_dequantizer_interface(gpu) -> None:
    assert HipDequantizer.supports(D.Q4_K) and not HipDequantizer.supports(10)
    assert HipDequantizer.geometry(D.Q6_K) == (256, 210)
    w = S.packed_weight(D.Q8_0, 4, 256, seed=1)
    got = host(HipDequantizer.dequantize(torch.from_numpy(w).cuda().reshape(-1, 34), D.Q8_0))
    assert np.array_equal(bits(got), bits(D.dequantize(D.Q8_0, w)))
