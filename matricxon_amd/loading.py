"""Load path: packed GGUF bytes from the host (the loader's read-only mmap) into HBM, still
packed, and packed row reordering on the device.

* `PackedUploader(device)`: host -> device copies through pinned staging buffers. Each chunk is
  copied from the source (pageable, typically the mmap) into a pinned buffer by a few host
  threads, then sent with an asynchronous copy on a copy stream while the next chunk is staged,
  so the host copy and the PCIe transfer overlap. The reference's `upload_packed`
  (app/architectures/device_packed.py:14-19) copies from pageable memory in one synchronous call.
* `upload(raw, n_rows, order=None)`: (n_rows, row_bytes) uint8 device tensor holding a copy of
  `raw` (never an alias); with `order`, row i is source row order[i], reordered on the device
  (`PackedRows.reordered`, app/gguf/packed_rows.py:24-28, and `unpermute_rope_rows`' use of it).
* `upload_experts(raw, num_experts, out_features)`: one device allocation for a packed MoE
  tensor (num_experts, out_features, row_bytes) and one (out_features, row_bytes) view per
  expert, for the per-expert modules of app/architectures/moe_experts.py:105-121.

Chunking (`plan_chunks`) is plain host arithmetic; the device work is copies and the row gather
kernel (`mxa_gather_rows`).
"""

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from matricxon_amd.gemm import HipGemm

DEFAULT_CHUNK = 32 << 20
DEFAULT_BUFFERS = 3
HOST_THREADS = 4


def plan_chunks(total: int, chunk: int) -> list[tuple[int, int]]:
    """(offset, length) pieces of [0, total), each at most `chunk` bytes, in order."""
    if total < 0 or chunk <= 0:
        raise ValueError("total must be >= 0 and chunk > 0")
    return [(off, min(chunk, total - off)) for off in range(0, total, chunk)]


def host_bytes(raw) -> np.ndarray:
    """A flat uint8 numpy view of bytes-like `raw` (memoryview, bytes, numpy array or CPU
    tensor), without copying where the source allows."""
    if isinstance(raw, torch.Tensor):
        if raw.device.type != "cpu":
            raise ValueError("raw must be host memory")
        return raw.detach().contiguous().reshape(-1).view(torch.uint8).numpy()
    if isinstance(raw, np.ndarray):
        return np.ascontiguousarray(raw).reshape(-1).view(np.uint8)
    return np.frombuffer(memoryview(raw).cast("B"), dtype=np.uint8)


class PackedUploader:
    """Staged host -> device copies of packed weights for one device (see the module doc)."""

    def __init__(self, device: torch.device | str = "cuda", chunk_bytes: int = DEFAULT_CHUNK,
                 n_buffers: int = DEFAULT_BUFFERS, host_threads: int = HOST_THREADS) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("PackedUploader copies to a GPU device")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        if chunk_bytes <= 0 or n_buffers < 2 or host_threads < 1:
            raise ValueError("chunk_bytes > 0, n_buffers >= 2 and host_threads >= 1 are required")
        self.chunk_bytes = chunk_bytes
        self._buffers = [torch.empty(chunk_bytes, dtype=torch.uint8, pin_memory=True)
                         for _ in range(n_buffers)]
        self._events: list[torch.cuda.Event | None] = [None] * n_buffers
        self._stream = torch.cuda.Stream(device=self.device)
        self._pool = ThreadPoolExecutor(max_workers=host_threads) if host_threads > 1 else None
        self._threads = host_threads

    def close(self) -> None:
        if self._pool is not None:
            self._pool.shutdown(wait=True)
            self._pool = None

    def __enter__(self) -> "PackedUploader":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def _stage(self, dst: np.ndarray, src: np.ndarray) -> None:
        """Host copy src -> dst (pinned), split over the host threads."""
        n = src.shape[0]
        if self._pool is None or n < (4 << 20):
            np.copyto(dst, src)
            return
        step = -(-n // self._threads)
        parts = [(i, min(n, i + step)) for i in range(0, n, step)]
        list(self._pool.map(lambda p: np.copyto(dst[p[0]:p[1]], src[p[0]:p[1]]), parts))

    def copy_into(self, dst: torch.Tensor, raw) -> torch.Tensor:
        """Copies host bytes `raw` into the contiguous uint8 device tensor `dst` (same byte
        count). The copies are ordered before later work on the caller's current stream."""
        src = host_bytes(raw)
        if dst.dtype != torch.uint8 or not dst.is_contiguous() or dst.device != self.device:
            raise ValueError("dst must be a contiguous uint8 tensor on the uploader's device")
        if dst.numel() != src.shape[0]:
            raise ValueError(f"dst holds {dst.numel()} bytes, source has {src.shape[0]}")
        flat = dst.reshape(-1)
        # the copy stream starts after work already queued on the caller's stream (dst's
        # allocation may be reused memory still being read there)
        caller = torch.cuda.current_stream(self.device)
        self._stream.wait_stream(caller)
        nb = len(self._buffers)
        for i, (off, n) in enumerate(plan_chunks(src.shape[0], self.chunk_bytes)):
            b = i % nb
            if self._events[b] is not None:
                self._events[b].synchronize()  # the copy that last read this buffer is done
            buf = self._buffers[b]
            self._stage(buf[:n].numpy(), src[off:off + n])
            with torch.cuda.stream(self._stream):
                flat[off:off + n].copy_(buf[:n], non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(self._stream)
            self._events[b] = ev
        caller.wait_stream(self._stream)
        dst.record_stream(self._stream)
        return dst

    def upload(self, raw, n_rows: int, order: torch.Tensor | None = None) -> torch.Tensor:
        """(n_rows, row_bytes) uint8 device copy of packed bytes `raw`; with `order`, row i of the
        result is row order[i] of `raw` (len(order) rows)."""
        src = host_bytes(raw)
        if n_rows <= 0 or src.shape[0] % n_rows:
            raise ValueError(f"{src.shape[0]} packed bytes don't split into {n_rows} equal rows")
        dst = torch.empty((n_rows, src.shape[0] // n_rows), dtype=torch.uint8, device=self.device)
        self.copy_into(dst, src)
        if order is None:
            return dst
        return HipGemm.get().gather_rows(dst, order)

    def upload_experts(self, raw, num_experts: int,
                       out_features: int) -> tuple[torch.Tensor, list[torch.Tensor]]:
        """(all experts (num_experts, out_features, row_bytes), [per-expert views])."""
        src = host_bytes(raw)
        if num_experts <= 0 or out_features <= 0 or src.shape[0] % (num_experts * out_features):
            raise ValueError(f"{src.shape[0]} packed bytes don't split into {num_experts} experts "
                             f"of {out_features} equal rows")
        rb = src.shape[0] // (num_experts * out_features)
        dst = torch.empty((num_experts, out_features, rb), dtype=torch.uint8, device=self.device)
        self.copy_into(dst, src)
        return dst, [dst[e] for e in range(num_experts)]
