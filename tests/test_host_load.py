"""Host-side logic of the load path (matricxon_amd/loading.py) on the CPU: chunk planning and the
byte views of the sources the loader hands over. The device copies and the row gather are
tested on the GPU (test_gpu_load.py)."""

import mmap

import numpy as np
import pytest
import torch

from matricxon_amd.loading import host_bytes, plan_chunks


@pytest.mark.parametrize("total,chunk", [(0, 8), (1, 8), (8, 8), (9, 8), (100, 7), (1 << 20, 4096)])
def test_plan_chunks_cover_in_order(total, chunk) -> None:
    parts = plan_chunks(total, chunk)
    assert sum(n for _, n in parts) == total
    assert all(0 < n <= chunk for _, n in parts)
    offs = [o for o, _ in parts]
    assert offs == sorted(offs) and all(o + n == nxt for (o, n), nxt in zip(parts, offs[1:]))


def test_plan_chunks_rejects_bad_sizes() -> None:
    with pytest.raises(ValueError):
        plan_chunks(10, 0)
    with pytest.raises(ValueError):
        plan_chunks(-1, 4)


def test_host_bytes_views(tmp_path) -> None:
    data = np.arange(1000, dtype=np.uint16)
    raw = data.tobytes()
    for src in (raw, memoryview(raw), data, torch.from_numpy(data.copy())):
        assert host_bytes(src).tobytes() == raw
    path = tmp_path / "w.bin"
    path.write_bytes(raw)
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        view = memoryview(mm)[100:900]  # a slice of the read-only mmap, as the loader passes
        hb = host_bytes(view)
        assert hb.tobytes() == raw[100:900] and np.shares_memory(hb, np.frombuffer(mm, np.uint8))
        del hb, view
    with pytest.raises(ValueError):
        host_bytes(torch.zeros(4, device="meta"))
