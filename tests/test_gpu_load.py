"""Load path on the GPU: staged host -> device uploads of packed bytes and the device row gather
(`mxa_gather_rows`), each checked byte for byte against numpy (`PackedRows.reordered`,
app/gguf/packed_rows.py:24-28, is `rows[order]` on the host)."""

import mmap

import numpy as np
import pytest
import torch

from matricxon_amd import synthetic as S
from matricxon_amd.device_packed import DevicePackedLinear, upload_packed
from matricxon_amd.gemm import HipGemm
from matricxon_amd.loading import PackedUploader
from oracle import dequant as D
from tests.test_gpu_kernels import host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def uploader():
    # small chunks and buffers so every test crosses several chunks and reuses each buffer
    with PackedUploader("cuda", chunk_bytes=1 << 20, n_buffers=2, host_threads=3) as up:
        yield up


@pytest.mark.parametrize("n_rows,row_bytes", [(1, 7), (3, 210), (1000, 2304), (4096, 1360),
                                              (333, 11760)])
def test_upload_bit_exact(gpu, uploader, n_rows, row_bytes) -> None:
    rng = np.random.default_rng(n_rows)
    raw = rng.integers(0, 256, n_rows * row_bytes, dtype=np.uint8)
    dev = uploader.upload(memoryview(raw), n_rows)
    assert dev.shape == (n_rows, row_bytes) and dev.device.type == "cuda"
    assert np.array_equal(host(dev).reshape(-1), raw)
    raw[:] = 0  # a copy, never an alias of the source
    assert host(dev).any() or n_rows * row_bytes < 8


def test_upload_from_mmap_and_reference_signature(gpu, tmp_path) -> None:
    """upload_packed(raw, n_rows, device) from a slice of a read-only mmap, above the size where
    the staged uploader takes over."""
    n, k = 8192, 4096
    w = S.packed_weight(D.Q4_K, n, k, seed=3)  # 18.9 MB
    path = tmp_path / "t.bin"
    path.write_bytes(b"\0" * 64 + w.tobytes())
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        view = memoryview(mm)[64:]
        dev = upload_packed(view, n, torch.device("cuda"))
        torch.cuda.synchronize()
        del view
    assert np.array_equal(host(dev), w.reshape(n, -1))
    small = upload_packed(w[:4].copy(), 4, torch.device("cuda"))  # the plain path
    assert np.array_equal(host(small), w.reshape(n, -1)[:4])


@pytest.mark.parametrize("row_bytes", [2304, 210, 136, 34, 7])
def test_gather_rows_matches_numpy(gpu, row_bytes) -> None:
    rng = np.random.default_rng(row_bytes)
    n_src = 517
    rows = rng.integers(0, 256, (n_src, row_bytes), dtype=np.uint8)
    order = torch.from_numpy(rng.permutation(n_src)[:300].astype(np.int64))
    order[5] = order[6]  # repeats are allowed
    got = HipGemm.get().gather_rows(torch.from_numpy(rows).cuda(), order)
    assert np.array_equal(host(got), rows[order.numpy()])


def test_gather_rows_rope_permutation_on_packed_rows(gpu, uploader) -> None:
    """The loader's use: `unpermute_rope_rows`' row order (app/architectures/layers.py:9-29)
    applied to packed attn_q bytes; the matmul on the reordered weight equals the original's
    output columns in that order."""
    n_head, head_dim, k = 8, 64, 1024
    n = n_head * head_dim
    w = S.packed_weight(D.Q4_K, n, k, seed=5)
    order = (torch.arange(n).reshape(n_head, head_dim // 2, 2).transpose(1, 2).reshape(-1))
    dev = uploader.upload(w, n, order=order)
    assert np.array_equal(host(dev), w.reshape(n, -1)[order.numpy()])
    x = torch.randn(3, k, device="cuda")
    base = DevicePackedLinear(uploader.upload(w, n), k, D.Q4_K, dtype=torch.float32)(x)
    perm = DevicePackedLinear(dev, k, D.Q4_K, dtype=torch.float32)(x)
    assert torch.equal(perm, base[:, order.cuda()])


def test_gather_rows_rejects_out_of_range(gpu) -> None:
    src = torch.zeros((4, 16), dtype=torch.uint8, device="cuda")
    with pytest.raises(IndexError):
        HipGemm.get().gather_rows(src, torch.tensor([0, 4]))
    with pytest.raises(IndexError):
        HipGemm.get().gather_rows(src, torch.tensor([-1]))
    assert HipGemm.get().gather_rows(src, torch.tensor([], dtype=torch.int64)).shape == (0, 16)


def test_upload_experts_views(gpu, uploader) -> None:
    """A packed MoE tensor (num_experts, out, row_bytes): one allocation, one view per expert,
    each equal to that expert's slice (app/architectures/moe_experts.py:105-121)."""
    e, n, k = 6, 96, 512
    w = np.concatenate([S.packed_weight(D.Q6_K, n, k, seed=i) for i in range(e)])
    all_dev, views = uploader.upload_experts(w, e, n)
    assert all_dev.shape == (e, n, w.size // (e * n)) and len(views) == e
    per = w.reshape(e, n, -1)
    for i, v in enumerate(views):
        assert v.data_ptr() == all_dev[i].data_ptr() and np.array_equal(host(v), per[i])
    x = torch.randn(2, k, device="cuda")
    y = DevicePackedLinear(views[3], k, D.Q6_K, dtype=torch.float32)(x)
    ref = DevicePackedLinear(torch.from_numpy(per[3].copy()).cuda(), k, D.Q6_K,
                             dtype=torch.float32)(x)
    assert torch.equal(y, ref)
    with pytest.raises(ValueError):
        uploader.upload_experts(w[:-1], e, n)
