"""Drop-in replacements for the reference's packed GPU modules
(app/architectures/device_packed.py:14-89) that compute with the HIP kernels instead of
dequantizing with torch ops and calling `F.linear`.

* `DevicePackedLinear(packed, in_features, ggml_type, bias=None, dtype=torch.bfloat16)`: same
  constructor, attributes (`out_features`, `in_features`, non-persistent `packed` buffer,
  `bias`) and `forward(x: (..., K)) -> (..., N)` in `dtype`, as the reference's
  (device_packed.py:22-63). The weight is never dequantized: one fused quantized matmul per call.
* `DevicePackedEmbedding(packed, embedding_dim, ggml_type, dtype)`: lookups expand only the
  requested rows (device_packed.py:66-84); `as_linear` shares the bytes with the tied output
  projection (device_packed.py:86-89).
* `upload_packed(raw, n_rows, device)`: packed bytes copied into a new device tensor of
  n_rows rows (device_packed.py:14-19).
* `HipDequantizer`: the `TorchDequantizer` interface (torch_dequant.py:221-236) on the kernels.

A bfloat16 layer (the reference's GPU dtype) reads bfloat16 x and writes bfloat16 y straight from
the kernels (`mxa_gemm_bf16`: each output the float32 result rounded as torch's cast), so a call is
one library call with no cast launches. An input that a fused producer
(`matricxon_amd.fused_ops.HipFusedOps`) just wrote comes with its Q8_K blocks;
`DevicePackedLinear` then runs the matmul alone on them.

Only Q8_0, Q4_K, Q6_K and IQ4_XS (with in_features % 256 == 0) are computed here; a loader
asks `HipDequantizer.supports` / `HipGemm.supports` and keeps the reference module for the rest.

`MATRICXON_GEMV_BACKEND` (app/config.py:123, "native" by default) picks the activation numerics of
`DevicePackedLinear`: "native" quantizes x to Q8_K as the reference's C kernels do; "numba" keeps x
in float32 for decode-sized calls (`mxa_gemv_f32`, the Numba GEMVs' numerics,
app/gguf/dequant/quantized_gemv.py:51-180) and, like the reference's QuantizedLinear prefill
(app/architectures/quantized_linear.py:101-106), dequantizes the weight transiently to the layer
dtype for larger calls.
"""

import os
import warnings

import numpy as np
import torch
from torch import nn

from matricxon_amd.fused_ops import HANDOFF
from matricxon_amd.gemm import HipGemm
from matricxon_amd.quant_types import GEOMETRY

_IQ4_XS = 23
GEMV_BACKENDS = ("native", "numba")
# "numba" backend: rows per call that take the fp32-activation GEMV; the reference's
# QuantizedLinear takes its GEMV only for one token (batch == 1 and seq_len == 1,
# app/architectures/quantized_linear.py:94-98)
F32_GEMV_MAX_ROWS = 1


def gemv_backend() -> str:
    """`MATRICXON_GEMV_BACKEND`, "native" when unset; ValueError for another value (the
    reference's settings accept only these two, app/config.py:123)."""
    value = os.environ.get("MATRICXON_GEMV_BACKEND", "native").strip().lower()
    if value not in GEMV_BACKENDS:
        raise ValueError(f"MATRICXON_GEMV_BACKEND must be one of {GEMV_BACKENDS}, got {value!r}")
    return value


_UPLOADERS: dict[torch.device, "PackedUploader"] = {}
STAGED_UPLOAD_MIN_BYTES = 16 << 20


def _host_nbytes(raw) -> int | None:
    """Bytes of a host source; None for a device tensor."""
    if isinstance(raw, torch.Tensor):
        return None if raw.device.type != "cpu" else raw.numel() * raw.element_size()
    return memoryview(raw).nbytes


def upload_packed(raw, n_rows: int, device: torch.device) -> torch.Tensor:
    """A fresh device tensor of shape (n_rows, row_bytes), dtype uint8, holding the packed bytes of
    `raw`; `raw` itself is never referenced afterwards.
    Host sources of 16 MiB or more go to a GPU through the pinned, overlapped staging of
    `matricxon_amd.loading.PackedUploader`."""
    device = torch.device(device)
    nbytes = _host_nbytes(raw)
    if device.type == "cuda" and nbytes is not None and nbytes >= STAGED_UPLOAD_MIN_BYTES:
        from matricxon_amd.loading import PackedUploader

        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        up = _UPLOADERS.get(device)
        if up is None:
            up = _UPLOADERS[device] = PackedUploader(device)
        return up.upload(raw, n_rows)
    if isinstance(raw, torch.Tensor):
        flat = raw.reshape(-1).to(torch.uint8)
    else:
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            flat = torch.frombuffer(memoryview(np.ascontiguousarray(raw)).cast("B"),
                                    dtype=torch.uint8)
    return flat.reshape(n_rows, -1).to(device, copy=True)


class HipDequantizer:
    """Which quant types dequantize on the device with the HIP kernels, and their geometry."""

    @staticmethod
    def supports(ggml_type: int) -> bool:
        return int(ggml_type) in GEOMETRY

    @staticmethod
    def geometry(ggml_type: int) -> tuple[int, int]:
        """`(block_size, type_size)` of `ggml_type`."""
        return GEOMETRY[int(ggml_type)]

    @staticmethod
    def dequantize(blocks: torch.Tensor, ggml_type: int) -> torch.Tensor:
        return HipGemm.get().dequantize(blocks, ggml_type)


class DevicePackedLinear(nn.Module):
    """`nn.Linear` whose weight stays quantized in device memory and is multiplied in place by
    the fused HIP kernels: x is quantized to Q8_K (IQ4_XS: kept in float32) and multiplied
    against the packed blocks with float32 accumulation, as the reference's native C kernel does
    (app/native/src/mx_gemm.c:123-194)."""

    def __init__(
        self,
        packed: torch.Tensor,
        in_features: int,
        ggml_type: int,
        bias: torch.Tensor | None = None,
        dtype: torch.dtype = torch.bfloat16,
        *,
        backend: str | None = None,
    ) -> None:
        super().__init__()
        gemm = HipGemm.get()
        if not gemm.supports(int(ggml_type), in_features):
            raise ValueError(
                f"no HIP kernel for GGML type {int(ggml_type)} with in_features={in_features}"
            )
        backend = gemv_backend() if backend is None else backend
        if backend not in GEMV_BACKENDS:
            raise ValueError(f"backend must be one of {GEMV_BACKENDS}, got {backend!r}")
        self.backend = backend
        self.out_features = packed.shape[0]
        self.in_features = in_features
        self._ggml_type = int(ggml_type)
        self._dtype = dtype
        self._type_size = HipDequantizer.geometry(ggml_type)[1]
        self._gemm = gemm
        self.register_buffer("packed", packed, persistent=False)
        self.bias = None if bias is None else nn.Parameter(bias.to(packed.device, dtype))

    @property
    def ggml_type(self) -> int:
        return self._ggml_type

    @property
    def dtype(self) -> torch.dtype:
        return self._dtype

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        k = self.in_features
        if self.backend == "numba":
            return self.finish(self._forward_f32(x.reshape(-1, k)), lead)
        # The reference casts x to the layer dtype before its matmul (device_packed.py:54).
        if x.dtype != self._dtype:
            x = x.to(self._dtype)
        bf16 = self._dtype == torch.bfloat16  # the kernels read and write bfloat16 themselves
        dev = self.packed.device
        n, big_n = x.numel() // k, self.out_features
        ws = HANDOFF.claim(x) if self._ggml_type != _IQ4_XS else None
        if ws is not None:  # x came from a fused producer that also wrote its Q8_K blocks
            y = torch.empty((n, big_n), dtype=torch.bfloat16 if bf16 else torch.float32, device=dev)
            self._gemm.matmul_q8k(self._ggml_type, self.packed, ws, None, y, n, big_n, k)
        elif bf16 and x.device == dev and n > 0:
            xb = x.reshape(n, k)
            if not xb.is_contiguous() or xb.data_ptr() % 16 != 0:
                xb = xb.clone(memory_format=torch.contiguous_format)
            y = torch.empty((n, big_n), dtype=torch.bfloat16, device=dev)
            self._gemm._gemm_bf16(self._ggml_type, self.packed, xb, y, n, big_n, k)
        elif bf16:
            y = self._gemm.matmul_bf16(self._ggml_type, self.packed, x.reshape(-1, k), big_n, k)
        else:
            y = self._gemm.matmul(self._ggml_type, self.packed, x.reshape(-1, k), big_n, k)
        return self.finish(y, lead)

    def _forward_f32(self, x2: torch.Tensor) -> torch.Tensor:
        """The "numba" backend, as the reference's QuantizedLinear without its native library
        (quantized_linear.py:94-106): one token goes through the fp32-activation GEMV on x cast
        straight to float32; more rows take a transient dequantization to the layer dtype and a
        matmul of x in that dtype. (M, N) float32."""
        k, n = self.in_features, self.out_features
        if x2.shape[0] <= F32_GEMV_MAX_ROWS:
            return self._gemm.gemv_f32(self._ggml_type, self.packed, x2.to(torch.float32), n, k)
        weight = self._gemm.dequantize(self.packed, self._ggml_type).reshape(n, k).to(self._dtype)
        y = (x2.to(self._dtype) @ weight.T).to(torch.float32)
        del weight
        return y

    def finish(self, y: torch.Tensor, lead: tuple[int, ...]) -> torch.Tensor:
        """Result rows (M, N), float32 or already the layer's dtype -> the layer's output (..., N)
        in its dtype, plus bias."""
        if y.dtype != self._dtype:
            y = y.to(self._dtype)
        y = y.reshape(*lead, self.out_features)
        return y if self.bias is None else y + self.bias


class DevicePackedEmbedding(nn.Module):
    """Token embeddings kept as packed GGUF rows in device memory. `forward` expands just the
    looked-up ids (one `mxa_dequant_rows` launch); `as_linear` reuses the same bytes as the tied
    output projection."""

    def __init__(
        self, packed: torch.Tensor, embedding_dim: int, ggml_type: int, dtype: torch.dtype
    ) -> None:
        super().__init__()
        gemm = HipGemm.get()
        if not gemm.supports_dequant_rows(int(ggml_type), embedding_dim):
            raise ValueError(f"no HIP row dequantizer for GGML type {int(ggml_type)}")
        self.num_embeddings = packed.shape[0]
        self.embedding_dim = embedding_dim
        self.dtype = dtype
        self._ggml_type = int(ggml_type)
        self._type_size = HipDequantizer.geometry(ggml_type)[1]
        self._gemm = gemm
        self.register_buffer("packed", packed, persistent=False)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        # torch indexing semantics of the reference's `self.packed[ids]` (device_packed.py:81-84):
        # negative ids count from the end. The wrap runs on the device (no host sync); an id
        # outside [-num_embeddings, num_embeddings) gives a row of NaN instead of an error.
        flat = ids.reshape(-1).to(torch.int64)
        flat = torch.where(flat < 0, flat + self.num_embeddings, flat)
        rows = self._gemm.dequant_rows(self._ggml_type, self.packed, flat, self.embedding_dim)
        return rows.reshape(*ids.shape, self.embedding_dim).to(self.dtype)

    def as_linear(self) -> DevicePackedLinear:
        return DevicePackedLinear(self.packed, self.embedding_dim, self._ggml_type,
                                  dtype=self.dtype)
