"""Python face of the HIP quantized matmul (libmatricxon_amd.so): y = x @ W.T for a packed GGUF
weight W that stays packed in device memory.

`HipGemm` mirrors the reference's `NativeGemm` (app/native/gemm.py:22-212): `configure` /
`active` / `supports` / `matmul` / `supports_dequant_rows` / `dequant_rows` / `take_stats`, with
the same argument meaning and the same error behaviour (a nonzero library status becomes a
`RuntimeError` naming the status and the type). The differences are the ones the device imposes:
the packed weight is a device uint8 tensor instead of an mmap'd memoryview, x and y live on that
device, and the call is asynchronous on torch's current HIP stream (no host sync).
"""

import logging

import torch

from matricxon_amd import _lib
from matricxon_amd.quant_types import GEOMETRY, GGMLType

logger = logging.getLogger(__name__)


_ERR_WORKSPACE = -2  # MXA_ERR_WORKSPACE
_IQ4_XS = int(GGMLType.IQ4_XS)
_FUSED_MAX_TOKENS_CAP = 4  # the clamp of mxa_set_fused_max_tokens
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """torch's current HIP stream on `device` as a raw handle: the value of
    `torch.cuda.current_stream(device).cuda_stream`, read without building a Stream object (that
    costs about 2 us of host time per call, a quarter of a decode GEMV's launch path)."""
    if _RAW_STREAM is None:
        return torch.cuda.current_stream(device).cuda_stream
    index = device.index
    return _RAW_STREAM(torch.cuda.current_device() if index is None else index)


def _al256(n: int) -> int:
    return (n + 255) & ~255


def q8k_bytes(m: int, k: int) -> int:
    """Bytes of the Q8_K activation layout mxa_quantize_q8_k writes for (m, k) floats:
    q int8 (m, k) | d float32 (m, k/256) | bsums int16 (m, k/256, 16), each 256-byte aligned."""
    nb = k // 256
    return _al256(m * k) + _al256(m * nb * 4) + _al256(m * nb * 32)


def q8k_views(workspace: torch.Tensor, m: int, k: int) -> tuple[torch.Tensor, torch.Tensor,
                                                                  torch.Tensor]:
    """(q int8 (M, K), d float32 (M, K/256), bsums int16 (M, K/256, 16)) views of the Q8_K part
    at the start of a workspace: q, then d, then bsums, each starting on a 256-byte boundary."""
    nb = k // 256
    q = workspace[: m * k].view(torch.int8).reshape(m, k)
    off = _al256(m * k)
    d = workspace[off : off + m * nb * 4].view(torch.float32).reshape(m, nb)
    off += _al256(m * nb * 4)
    bs = workspace[off : off + m * nb * 32].view(torch.int16).reshape(m, nb, 16)
    return q, d, bs


def _require_device_tensor(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a tensor on a HIP device, got {getattr(t, 'device', t)}")


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """`t`, or a copy of it when its data does not start on a 16-byte boundary (the kernels read
    activations as 16-byte vectors; a view into the middle of a tensor may start anywhere)."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


class HipGemm:
    _active: "HipGemm | None" = None

    def __init__(self) -> None:
        self._lib = _lib.load()
        self.build_info = self._lib.mxa_build_info().decode()
        self._calls = 0
        self._fallback_types_logged: set[int] = set()

    # -- lifecycle (NativeGemm.configure / active, app/native/gemm.py:63-84) --------------------
    @classmethod
    def configure(cls, backend: str = "hip") -> None:
        """Loads the library once at startup. Unlike the reference's C build there is no fallback
        to hide a failure behind: a missing library raises `LibraryMissingError`."""
        cls._active = None
        if backend != "hip":
            return
        cls._active = cls()
        logger.info("HIP quantized kernels enabled: %s", cls._active.build_info)

    @classmethod
    def active(cls) -> "HipGemm | None":
        return cls._active

    @classmethod
    def get(cls) -> "HipGemm":
        """The configured instance, configuring on first use."""
        if cls._active is None:
            cls.configure("hip")
        return cls._active

    # -- capability queries ---------------------------------------------------------------------
    def supports(self, ggml_type: int, in_features: int) -> bool:
        supported = bool(self._lib.mxa_supports(int(ggml_type), int(in_features)))
        if not supported and int(ggml_type) not in self._fallback_types_logged:
            self._fallback_types_logged.add(int(ggml_type))
            logger.info("no HIP kernel for GGML type %d (in_features=%d)", int(ggml_type),
                        in_features)
        return supported

    def supports_dequant_rows(self, ggml_type: int, row_width: int) -> bool:
        """Whether `dequant_rows` handles (type, row_width) (`mx_supports_dequant_rows`,
        app/native/gemm.py:105-109): the four types here, row_width a multiple of 256."""
        return bool(self._lib.mxa_supports_dequant_rows(int(ggml_type), int(row_width)))

    def set_fused_max_tokens(self, n_tokens: int) -> None:
        """Up to this many tokens per call a K-quant / Q8_0 matmul runs on the decode kernel, which
        quantizes x itself; more tokens quantize into a workspace and run on the matrix cores
        (`NativeGemm.set_fused_max_tokens`, app/native/gemm.py:156-159). Clamped to [0, 4]; both
        kernels give the same bits, so only the speed crossover moves. Process-wide."""
        self._lib.mxa_set_fused_max_tokens(int(n_tokens))

    @property
    def fused_max_tokens(self) -> int:
        return int(self._lib.mxa_fused_max_tokens())

    def row_bytes(self, ggml_type: int, in_features: int) -> int:
        return int(self._lib.mxa_row_bytes(int(ggml_type), int(in_features)))

    def workspace_bytes(self, ggml_type: int, n_tokens: int, in_features: int) -> int:
        return int(self._lib.mxa_workspace_bytes(int(ggml_type), int(n_tokens), int(in_features)))

    # -- stats (NativeGemm.record / take_stats, app/native/gemm.py:161-171) ---------------------
    def record(self, seconds: float = 0.0) -> None:
        self._calls += 1

    def take_stats(self) -> tuple[int, float]:
        """(calls, 0.0) since the last call: launches are asynchronous, so host time is not the
        kernel time; per-kernel time comes from HIP events or rocprofv3."""
        stats = (self._calls, 0.0)
        self._calls = 0
        return stats

    # -- compute --------------------------------------------------------------------------------
    def _check(self, status: int, what: str, ggml_type: int) -> None:
        if status != 0:
            detail = self._lib.mxa_last_error().decode()
            raise RuntimeError(
                f"{what} failed with status {status} for type {ggml_type}"
                + (f": {detail}" if detail else "")
            )

    def _check_packed(self, ggml_type: int, packed: torch.Tensor, out_features: int,
                      in_features: int) -> None:
        _require_device_tensor("packed", packed)
        expected = (out_features, self.row_bytes(ggml_type, in_features))
        if packed.dtype != torch.uint8 or tuple(packed.shape) != expected:
            raise ValueError(
                f"packed must be uint8 {expected} for type {ggml_type}, got "
                f"{packed.dtype} {tuple(packed.shape)}"
            )
        if not packed.is_contiguous():
            raise ValueError("packed rows must be contiguous")

    def matmul(self, ggml_type: int, packed: torch.Tensor, x: torch.Tensor, out_features: int,
               in_features: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """`x`: (n_tokens, in_features), any float dtype, on packed's device. Returns
        (n_tokens, out_features) float32 (written into `out` when given)."""
        ggml_type = int(ggml_type)
        if not self.supports(ggml_type, in_features):
            raise RuntimeError(f"mxa_gemm failed with status -1 for type {ggml_type}")
        self._check_packed(ggml_type, packed, out_features, in_features)
        x32 = _aligned16(x.detach().reshape(-1, in_features).to(device=packed.device,
                                                                dtype=torch.float32).contiguous())
        n_tokens = x32.shape[0]
        if out is None:
            out = torch.empty((n_tokens, out_features), dtype=torch.float32, device=packed.device)
        elif out.shape != (n_tokens, out_features) or out.dtype != torch.float32 or \
                not out.is_contiguous() or out.device != packed.device:
            raise ValueError("out must be a contiguous float32 (n_tokens, out_features) tensor")
        if n_tokens == 0:
            return out
        ws_bytes = self.workspace_bytes(ggml_type, n_tokens, in_features)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=packed.device)
        status = self._lib.mxa_gemm(ggml_type, packed.data_ptr(), x32.data_ptr(), out.data_ptr(),
                                    n_tokens, out_features, in_features, ws.data_ptr(), ws_bytes,
                                    _stream(packed.device))
        self._check(status, "mxa_gemm", ggml_type)
        self._calls += 1
        return out

    def matmul_bf16(self, ggml_type: int, packed: torch.Tensor, x: torch.Tensor,
                    out_features: int, in_features: int,
                    out: torch.Tensor | None = None) -> torch.Tensor:
        """`matmul` for a bfloat16 layer (`mxa_gemm_bf16`): x (n_tokens, in_features) is taken as
        bfloat16 (cast first if it is not) and the result (n_tokens, out_features) is bfloat16, each
        value the float32 result rounded to nearest even as torch's cast rounds it. One library
        call, no cast launches."""
        ggml_type = int(ggml_type)
        if not self.supports(ggml_type, in_features):
            raise RuntimeError(f"mxa_gemm_bf16 failed with status -1 for type {ggml_type}")
        self._check_packed(ggml_type, packed, out_features, in_features)
        xb = x.detach().reshape(-1, in_features)
        if xb.dtype != torch.bfloat16 or xb.device != packed.device:
            xb = xb.to(device=packed.device, dtype=torch.bfloat16)
        xb = _aligned16(xb.contiguous())
        n_tokens = xb.shape[0]
        if out is None:
            out = torch.empty((n_tokens, out_features), dtype=torch.bfloat16, device=packed.device)
        elif out.shape != (n_tokens, out_features) or out.dtype != torch.bfloat16 or \
                not out.is_contiguous() or out.device != packed.device:
            raise ValueError("out must be a contiguous bfloat16 (n_tokens, out_features) tensor")
        if n_tokens == 0:
            return out
        self._gemm_bf16(ggml_type, packed, xb, out, n_tokens, out_features, in_features)
        return out

    def _gemm_bf16(self, ggml_type: int, packed: torch.Tensor, xb: torch.Tensor,
                   out: torch.Tensor, n_tokens: int, out_features: int, in_features: int) -> None:
        """The library call of `matmul_bf16` on checked operands: xb contiguous bfloat16 on
        packed's device, 16-byte aligned; out contiguous bfloat16. A decode-sized K-quant or Q8_0
        call is first made with no workspace: the kernel that reads bfloat16 x takes it in one
        launch, and any call it does not take returns MXA_ERR_WORKSPACE having launched nothing,
        to be made again with the workspace."""
        stream = _stream(packed.device)
        if ggml_type != _IQ4_XS and n_tokens <= _FUSED_MAX_TOKENS_CAP:
            status = self._lib.mxa_gemm_bf16(ggml_type, packed.data_ptr(), xb.data_ptr(),
                                             out.data_ptr(), n_tokens, out_features, in_features,
                                             None, 0, stream)
            if status != _ERR_WORKSPACE:
                self._check(status, "mxa_gemm_bf16", ggml_type)
                self._calls += 1
                return
        ws_bytes = self._lib.mxa_workspace_bytes_bf16(ggml_type, n_tokens, in_features)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=packed.device)
        status = self._lib.mxa_gemm_bf16(ggml_type, packed.data_ptr(), xb.data_ptr(),
                                         out.data_ptr(), n_tokens, out_features, in_features,
                                         ws.data_ptr(), ws_bytes, stream)
        self._check(status, "mxa_gemm_bf16", ggml_type)
        self._calls += 1

    def gemv_f32(self, ggml_type: int, packed: torch.Tensor, x: torch.Tensor, out_features: int,
                 in_features: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """`matmul` with x kept in float32 (never quantized to Q8_K), the numerics of the
        reference's fp32-activation GEMVs (app/gguf/dequant/quantized_gemv.py:51-180). Meant for
        decode-sized calls: the kernel takes four activation rows per pass over the weight.
        `x`: (n_tokens, in_features); returns (n_tokens, out_features) float32."""
        ggml_type = int(ggml_type)
        if not self.supports(ggml_type, in_features):
            raise RuntimeError(f"mxa_gemv_f32 failed with status -1 for type {ggml_type}")
        self._check_packed(ggml_type, packed, out_features, in_features)
        x32 = _aligned16(x.detach().reshape(-1, in_features).to(device=packed.device,
                                                                dtype=torch.float32).contiguous())
        n_tokens = x32.shape[0]
        if out is None:
            out = torch.empty((n_tokens, out_features), dtype=torch.float32, device=packed.device)
        elif out.shape != (n_tokens, out_features) or out.dtype != torch.float32 or \
                not out.is_contiguous() or out.device != packed.device:
            raise ValueError("out must be a contiguous float32 (n_tokens, out_features) tensor")
        if n_tokens == 0:
            return out
        status = self._lib.mxa_gemv_f32(ggml_type, packed.data_ptr(), x32.data_ptr(),
                                        out.data_ptr(), n_tokens, out_features, in_features,
                                        _stream(packed.device))
        self._check(status, "mxa_gemv_f32", ggml_type)
        self._calls += 1
        return out

    def matmul_q8k(self, ggml_type: int, packed: torch.Tensor, workspace: torch.Tensor,
                   x: torch.Tensor | None, out: torch.Tensor, n_tokens: int, out_features: int,
                   in_features: int) -> torch.Tensor:
        """The matmul kernel alone on activations already quantized into `workspace` (by
        `quantize_into`); `x` (float32, contiguous) is read only for IQ4_XS. `out` float32, or
        bfloat16 for a K-quant / Q8_0 weight (each value rounded as torch's cast)."""
        ggml_type = int(ggml_type)
        if out.dtype == torch.bfloat16:
            status = self._lib.mxa_gemm_q8k_bf16(ggml_type, packed.data_ptr(), out.data_ptr(),
                                                 n_tokens, out_features, in_features,
                                                 workspace.data_ptr(), workspace.numel(),
                                                 _stream(packed.device))
            self._check(status, "mxa_gemm_q8k_bf16", ggml_type)
            return out
        status = self._lib.mxa_gemm_q8k(ggml_type, packed.data_ptr(),
                                        None if x is None else x.data_ptr(), out.data_ptr(),
                                        n_tokens, out_features, in_features,
                                        workspace.data_ptr(), workspace.numel(),
                                        _stream(packed.device))
        self._check(status, "mxa_gemm_q8k", ggml_type)
        return out

    def quantize_into(self, x: torch.Tensor, workspace: torch.Tensor) -> None:
        """Q8_K activations of x (M, K) float32 or bfloat16, contiguous, into `workspace` (uint8,
        at least `q8k_bytes(M, K)` bytes)."""
        m, k = x.shape
        fn = self._lib.mxa_quantize_q8_k_bf16 if x.dtype == torch.bfloat16 else \
            self._lib.mxa_quantize_q8_k
        status = fn(x.data_ptr(), m, k, workspace.data_ptr(), workspace.numel(), _stream(x.device))
        self._check(status, "mxa_quantize_q8_k", 15)

    def matmul_multi(self, items: list[tuple[int, torch.Tensor, int]], x: torch.Tensor,
                     out: torch.Tensor | None = None, bf16: bool = False) -> list[torch.Tensor]:
        """`items`: (ggml_type, packed, out_features) per weight sharing input `x`
        (n_tokens, in_features): one activation quantization, one float32 output per weight,
        as `MultiGemmPlan.run` (app/native/gemm_multi.py:46-61) returns them. For up to 16 tokens
        and K-quant / Q8_0 weights of up to 16 blocks per row this is a single matmul launch.
        `out`, if given, is the (n_tokens, sum of out_features) result buffer the outputs are
        views of. `bf16`: x taken as bfloat16 and the outputs bfloat16 (`mxa_gemm_multi_bf16`,
        a bfloat16 layer's projections)."""
        import ctypes

        if not 1 <= len(items) <= 4:
            raise ValueError("matmul_multi takes 1 to 4 weights")
        in_features = x.shape[-1]
        device = items[0][1].device
        for t, p, o in items:
            if not self.supports(t, in_features):
                raise RuntimeError(f"mxa_gemm_multi failed with status -1 for type {t}")
            self._check_packed(int(t), p, o, in_features)
            if p.device != device:
                raise ValueError("all packed weights must be on one device")
        dtype = torch.bfloat16 if bf16 else torch.float32
        xc = _aligned16(x.detach().reshape(-1, in_features).to(device=device, dtype=dtype)
                        .contiguous())
        n_tokens = xc.shape[0]
        outs = [int(o) for _, _, o in items]
        if out is None:
            y = torch.empty((n_tokens, sum(outs)), dtype=dtype, device=device)
        else:
            if (out.dtype != dtype or out.device != device or not out.is_contiguous()
                    or tuple(out.shape) != (n_tokens, sum(outs))):
                raise ValueError(f"out must be a contiguous {dtype} (n_tokens, sum of "
                                 "out_features) tensor on the weights' device")
            y = out
        # the Q8_K part and the IQ4_XS part(s) are separate regions of one workspace
        size_of = self._lib.mxa_workspace_bytes_bf16 if bf16 else self._lib.mxa_workspace_bytes
        need = {False: 0, True: 0}
        for t, _, _ in items:
            is_iq4 = int(t) == 23
            need[is_iq4] = max(need[is_iq4], int(size_of(int(t), n_tokens, in_features)))
        ws_bytes = need[False] + need[True]
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
        n = len(items)
        types = (ctypes.c_int * n)(*[int(t) for t, _, _ in items])
        ptrs = (ctypes.c_void_p * n)(*[p.data_ptr() for _, p, _ in items])
        couts = (ctypes.c_int * n)(*outs)
        fn = self._lib.mxa_gemm_multi_bf16 if bf16 else self._lib.mxa_gemm_multi
        status = fn(n, types, ptrs, couts, xc.data_ptr(), y.data_ptr(), n_tokens, in_features,
                    ws.data_ptr(), ws_bytes, _stream(device))
        self._check(status, "mxa_gemm_multi", int(items[0][0]))
        self._calls += 1
        return list(torch.split(y, outs, dim=-1))

    # -- fused producers: FusedOps.rms_norm / silu_mul (app/architectures/layers.py:53-81) whose
    #    result is also written as Q8_K for the projections that consume it ----------------------
    def rms_norm_q8k(self, x: torch.Tensor, weight: torch.Tensor, eps: float,
                     want_out: bool = True) -> tuple[torch.Tensor | None, torch.Tensor]:
        """RMSNorm of the rows of x (..., K) on the device with `weight` (K,), in float32:
        (out float32 (M, K) or None, workspace) where the workspace holds the Q8_K blocks of out,
        ready for `matmul_multi_q8k` / `matmul_q8k`. K must be a multiple of 256."""
        _require_device_tensor("x", x)
        if x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16:
            return self._rms_norm_q8k_bf16(x, weight, eps, want_out)
        x32 = x.detach().to(torch.float32).reshape(-1, x.shape[-1]).contiguous()
        w32 = weight.detach().to(device=x.device, dtype=torch.float32).contiguous()
        m, k = x32.shape
        if w32.shape != (k,):
            raise ValueError("weight must have shape (K,) for x (..., K)")
        out = torch.empty_like(x32) if want_out else None
        ws = torch.empty(q8k_bytes(m, k), dtype=torch.uint8, device=x.device)
        status = self._lib.mxa_rms_norm_q8_k(x32.data_ptr(), w32.data_ptr(), float(eps), m, k,
                                             None if out is None else out.data_ptr(),
                                             ws.data_ptr(), ws.numel(), _stream(x.device))
        self._check(status, "mxa_rms_norm_q8_k", 15)
        return out, ws

    def _rms_norm_q8k_bf16(self, x: torch.Tensor, weight: torch.Tensor, eps: float,
                           want_out: bool) -> tuple[torch.Tensor | None, torch.Tensor]:
        """`rms_norm_q8k` of a bfloat16 layer (x and weight bfloat16): the reference's torch steps
        for those dtypes (app/architectures/layers.py:77-81), out bfloat16 (M, K), and the Q8_K
        blocks of out. K up to 16384."""
        k = x.shape[-1]
        xb = _aligned16(x.detach().reshape(-1, k).contiguous())
        wb = _aligned16(weight.detach().to(x.device).contiguous())
        m = xb.shape[0]
        if wb.shape != (k,):
            raise ValueError("weight must have shape (K,) for x (..., K)")
        out = torch.empty_like(xb) if want_out else None
        ws = torch.empty(q8k_bytes(m, k), dtype=torch.uint8, device=x.device)
        status = self._lib.mxa_rms_norm_q8_k_bf16(xb.data_ptr(), wb.data_ptr(), float(eps), m, k,
                                                  None if out is None else out.data_ptr(),
                                                  ws.data_ptr(), ws.numel(), _stream(x.device))
        self._check(status, "mxa_rms_norm_q8_k_bf16", 15)
        return out, ws

    def silu_mul_q8k(self, gate: torch.Tensor, up: torch.Tensor,
                     want_out: bool = True) -> tuple[torch.Tensor | None, torch.Tensor]:
        """silu(gate) * up over (..., K) on the device, in float32: (out (M, K) or None,
        workspace with the Q8_K blocks of out), the down projection's input. K must be a multiple
        of 256. Two float32 (M, K) views with unit column stride and one common row stride (the
        halves of a gate|up output) are read in place."""
        _require_device_tensor("gate", gate)
        if gate.shape != up.shape or gate.dim() == 0:
            raise ValueError("gate and up must have the same shape")
        k = gate.shape[-1]
        g2, u2 = gate.detach().reshape(-1, k), up.detach().reshape(-1, k)
        if g2.dtype == u2.dtype == torch.bfloat16:
            return self._silu_mul_q8k_bf16(g2, u2, want_out)
        if not (g2.dtype == u2.dtype == torch.float32 and u2.device == g2.device
                and g2.stride(-1) == u2.stride(-1) == 1 and g2.stride(0) == u2.stride(0)
                and g2.stride(0) >= k):
            g2 = g2.to(torch.float32).contiguous()
            u2 = u2.to(device=g2.device, dtype=torch.float32).contiguous()
        m = g2.shape[0]
        out = torch.empty((m, k), dtype=torch.float32, device=g2.device) if want_out else None
        ws = torch.empty(q8k_bytes(m, k), dtype=torch.uint8, device=g2.device)
        status = self._lib.mxa_silu_mul_q8_k(g2.data_ptr(), u2.data_ptr(), g2.stride(0), m, k,
                                             None if out is None else out.data_ptr(),
                                             ws.data_ptr(), ws.numel(), _stream(g2.device))
        self._check(status, "mxa_silu_mul_q8_k", 15)
        return out, ws

    def _silu_mul_q8k_bf16(self, g2: torch.Tensor, u2: torch.Tensor,
                           want_out: bool) -> tuple[torch.Tensor | None, torch.Tensor]:
        """`silu_mul_q8k` of bfloat16 (M, K) gate and up (read in place when they share a row
        stride, a multiple of 4, with unit column stride and 8-byte aligned data, as the halves of a
        gate|up output): torch's steps for bfloat16 tensors, out bfloat16."""
        k = g2.shape[-1]
        if not (u2.device == g2.device and g2.stride(-1) == u2.stride(-1) == 1
                and g2.stride(0) == u2.stride(0) and g2.stride(0) >= k and g2.stride(0) % 4 == 0
                and g2.data_ptr() % 8 == 0 and u2.data_ptr() % 8 == 0):
            g2 = _aligned16(g2.contiguous())
            u2 = _aligned16(u2.to(g2.device).contiguous())
        m = g2.shape[0]
        out = torch.empty((m, k), dtype=torch.bfloat16, device=g2.device) if want_out else None
        ws = torch.empty(q8k_bytes(m, k), dtype=torch.uint8, device=g2.device)
        status = self._lib.mxa_silu_mul_q8_k_bf16(g2.data_ptr(), u2.data_ptr(), g2.stride(0), m, k,
                                                  None if out is None else out.data_ptr(),
                                                  ws.data_ptr(), ws.numel(), _stream(g2.device))
        self._check(status, "mxa_silu_mul_q8_k_bf16", 15)
        return out, ws

    def matmul_moe(self, ggml_type: int, experts: torch.Tensor, x: torch.Tensor | None,
                   offsets: torch.Tensor, max_rows_per_expert: int, out_features: int,
                   in_features: int, workspace: torch.Tensor | None = None,
                   out: torch.Tensor | None = None,
                   out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Grouped projection of packed MoE experts (`mxa_gemm_moe`), one launch for all of
        them: `experts` (n_experts, out_features, row_bytes) uint8 on the device; rows
        [offsets[e], offsets[e + 1]) of `x` (n_rows, in_features) go through expert e
        (`offsets`: int32 on the device, n_experts + 1 ascending values from 0 to n_rows, so no
        host sync). x None: `workspace` already holds the Q8_K activations of the n_rows rows.
        Returns (n_rows, out_features) float32; each row equals `matmul` of that row alone bit
        for bit. `out_dtype` bfloat16 writes the result as bfloat16, each value the float32
        result rounded as torch's cast rounds it (`mxa_gemm_moe_bf16`). Replaces the per-expert
        calls of QuantizedMoEExperts.forward (app/architectures/moe_experts.py:81-88)."""
        ggml_type = int(ggml_type)
        _require_device_tensor("experts", experts)
        device = experts.device
        rb = self.row_bytes(ggml_type, in_features)
        if experts.dtype != torch.uint8 or experts.dim() != 3 or \
                tuple(experts.shape[1:]) != (out_features, rb) or not experts.is_contiguous():
            raise ValueError(f"experts must be contiguous uint8 (n_experts, {out_features}, {rb})")
        n_experts = experts.shape[0]
        if offsets.dtype != torch.int32 or offsets.shape != (n_experts + 1,) or \
                offsets.device != device:
            raise ValueError(f"offsets must be int32 ({n_experts + 1},) on {device}")
        x32 = None
        if x is not None:
            x32 = _aligned16(x.detach().reshape(-1, in_features).to(device=device,
                                                                    dtype=torch.float32).contiguous())
            n_rows = x32.shape[0]
        elif workspace is None:
            raise ValueError("matmul_moe needs x or a workspace holding its Q8_K activations")
        else:
            n_rows = out.shape[0] if out is not None else -1
            if n_rows < 0:
                raise ValueError("matmul_moe on a prequantized workspace needs `out` (n_rows rows)")
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"out_dtype must be float32 or bfloat16, not {out_dtype}")
        if out is None:
            out = torch.empty((n_rows, out_features), dtype=out_dtype, device=device)
        elif out.shape != (n_rows, out_features) or out.dtype != out_dtype or \
                not out.is_contiguous() or out.device != device:
            raise ValueError(f"out must be a contiguous {out_dtype} (n_rows, out_features) tensor")
        if n_rows == 0:
            return out
        if workspace is None and ggml_type != 23:  # IQ4_XS multiplies the float rows: none
            workspace = torch.empty(q8k_bytes(n_rows, in_features), dtype=torch.uint8,
                                    device=device)
        name = "mxa_gemm_moe_bf16" if out_dtype == torch.bfloat16 else "mxa_gemm_moe"
        status = getattr(self._lib, name)(
            ggml_type, experts.data_ptr(), rb * out_features, n_experts,
            None if x32 is None else x32.data_ptr(), offsets.data_ptr(), n_rows,
            max(1, min(int(max_rows_per_expert), n_rows)), out.data_ptr(), out_features,
            in_features, None if workspace is None else workspace.data_ptr(),
            0 if workspace is None else workspace.numel(), _stream(device))
        self._check(status, name, ggml_type)
        self._calls += 1
        return out

    def matmul_moe_pairs(self, ggml_type: int, experts: torch.Tensor, ids: torch.Tensor,
                         x: torch.Tensor | None, out_features: int, in_features: int,
                         workspace: torch.Tensor | None = None, x_rows: int | None = None,
                         out_dtype: torch.dtype = torch.float32) -> torch.Tensor | None:
        """One token's routed experts in one launch (`mxa_gemm_moe_pairs`): row p of the result
        (n_pairs, out_features) is expert ids[p] of `experts` (n_experts, out_features,
        row_bytes) times row p of `x` (n_pairs rows) or the single row of `x` (one row shared by
        all pairs). `ids`: int32 on the device, so no host sync. `out_dtype` bfloat16: x is read
        as bfloat16 and the result written as bfloat16, each value the float32 result rounded as
        torch's cast rounds it (`mxa_gemm_moe_pairs_bf16`). x None: `workspace` already holds the
        Q8_K blocks of `x_rows` rows (a producer's output). None when the shape does not suit the
        launch (the caller takes `matmul_moe`). Replaces the per-expert calls of
        QuantizedMoEExperts.forward for one token (app/architectures/moe_experts.py:81-88)."""
        ggml_type = int(ggml_type)
        _require_device_tensor("experts", experts)
        device = experts.device
        rb = self.row_bytes(ggml_type, in_features)
        if experts.dtype != torch.uint8 or experts.dim() != 3 or \
                tuple(experts.shape[1:]) != (out_features, rb) or not experts.is_contiguous():
            raise ValueError(f"experts must be contiguous uint8 (n_experts, {out_features}, {rb})")
        n_pairs = ids.numel()
        if ids.dtype != torch.int32 or ids.device != device or not ids.is_contiguous():
            raise ValueError(f"ids must be contiguous int32 on {device}")
        if out_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"out_dtype must be float32 or bfloat16, not {out_dtype}")
        bf16 = out_dtype == torch.bfloat16
        if x is None:
            if workspace is None or x_rows is None:
                raise ValueError("x None needs the workspace holding the Q8_K blocks and x_rows")
            xx = None
        else:
            xx = _aligned16(x.detach().reshape(-1, in_features).to(
                device=device, dtype=torch.bfloat16 if bf16 else torch.float32).contiguous())
            x_rows = xx.shape[0]
        if x_rows not in (1, n_pairs):
            raise ValueError(f"x must have 1 or {n_pairs} rows, not {x_rows}")
        if workspace is None:
            workspace = torch.empty(q8k_bytes(x_rows, in_features), dtype=torch.uint8, device=device)
        out = torch.empty((n_pairs, out_features), dtype=out_dtype, device=device)
        name = "mxa_gemm_moe_pairs_bf16" if bf16 else "mxa_gemm_moe_pairs"
        status = getattr(self._lib, name)(
            ggml_type, experts.data_ptr(), rb * out_features, experts.shape[0], ids.data_ptr(),
            n_pairs, None if xx is None else xx.data_ptr(), x_rows, out.data_ptr(), out_features,
            in_features, workspace.data_ptr(), workspace.numel(), _stream(device))
        if status == -1:
            return None
        self._check(status, name, ggml_type)
        self._calls += 1
        return out

    MOE_ROUTE_MAX_EXPERTS = 256
    MOE_ROUTE_MAX_PAIRS = 1 << 20

    def moe_route(self, top_k_idx: torch.Tensor, num_experts: int
                  ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """The routing of MoE (token, slot) pairs in one launch (`mxa_moe_route`), no host sync:
        (offsets (num_experts + 1,), pair_tok (n_pairs,), rows (n_tokens, top_k), ids32 (n_tokens,
        top_k)), all int32 on top_k_idx's device. `pair_tok` lists each pair's token in expert
        order (tokens ascending within an expert: a stable sort of the flattened ids clamped into
        [0, num_experts)), `rows[t, k]` is the place of pair (t, k) in that order, `offsets`
        delimits each expert's pairs and `ids32` is top_k_idx converted to int32. `top_k_idx`:
        (n_tokens, top_k) int32 or int64 on the device; num_experts <= MOE_ROUTE_MAX_EXPERTS and
        n_tokens * top_k <= MOE_ROUTE_MAX_PAIRS (else ValueError)."""
        _require_device_tensor("top_k_idx", top_k_idx)
        if top_k_idx.dim() != 2 or top_k_idx.dtype not in (torch.int32, torch.int64):
            raise ValueError("top_k_idx must be an int32 or int64 (n_tokens, top_k) tensor")
        n_tokens, top_k = top_k_idx.shape
        if not (1 <= num_experts <= self.MOE_ROUTE_MAX_EXPERTS) or n_tokens < 1 or top_k < 1 or \
                n_tokens * top_k > self.MOE_ROUTE_MAX_PAIRS:
            raise ValueError(f"mxa_moe_route takes 1..{self.MOE_ROUTE_MAX_EXPERTS} experts and "
                             f"1..{self.MOE_ROUTE_MAX_PAIRS} pairs")
        ids = top_k_idx.contiguous()
        device = ids.device
        offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=device)
        pair_tok = torch.empty(n_tokens * top_k, dtype=torch.int32, device=device)
        rows = torch.empty((n_tokens, top_k), dtype=torch.int32, device=device)
        ids32 = torch.empty((n_tokens, top_k), dtype=torch.int32, device=device)
        status = self._lib.mxa_moe_route(ids.data_ptr(), int(ids.dtype == torch.int64), n_tokens,
                                         top_k, int(num_experts), offsets.data_ptr(),
                                         pair_tok.data_ptr(), rows.data_ptr(), ids32.data_ptr(),
                                         _stream(device))
        self._check(status, "mxa_moe_route", 0)
        return offsets, pair_tok, rows, ids32

    def moe_combine(self, down: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                    rows: torch.Tensor | None = None, round_bf16: bool = False) -> torch.Tensor:
        """The weighted combine of MoE expert outputs in one launch (`mxa_moe_combine`): row t of
        the result (n_tokens, n_embd) float32 adds, in ascending expert id of token t's slots
        (`ids` (n_tokens, top_k) int32; equal ids in slot order), down row rows[t, k] (`rows`
        int32 like `ids`, or None for row t * top_k + k) times weights[t, k] (float32), from a
        float zero; `round_bf16` rounds each down value to bfloat16 first, as the module's cast
        to a bfloat16 layer dtype does. The combine of QuantizedMoEExperts.forward
        (app/architectures/moe_experts.py:81-88), bit for bit."""
        _require_device_tensor("down", down)
        device = down.device
        if down.dtype != torch.float32 or down.dim() != 2 or not down.is_contiguous():
            raise ValueError("down must be a contiguous float32 (rows, n_embd) tensor")
        if ids.dim() != 2:
            raise ValueError("ids must be (n_tokens, top_k)")
        n_tokens, top_k = ids.shape
        for name, t, dt in (("ids", ids, torch.int32), ("weights", weights, torch.float32)) + (
                (("rows", rows, torch.int32),) if rows is not None else ()):
            if t.dtype != dt or t.device != device or not t.is_contiguous() or \
                    tuple(t.shape) != (n_tokens, top_k):
                raise ValueError(f"{name} must be a contiguous {dt} ({n_tokens}, {top_k}) tensor "
                                 f"on {device}")
        out = torch.empty((n_tokens, down.shape[1]), dtype=torch.float32, device=device)
        status = self._lib.mxa_moe_combine(
            down.data_ptr(), rows.data_ptr() if rows is not None else None, ids.data_ptr(),
            weights.data_ptr(), n_tokens, top_k, down.shape[1], int(bool(round_bf16)),
            out.data_ptr(), _stream(device))
        self._check(status, "mxa_moe_combine", 0)
        self._calls += 1
        return out

    def matmul_multi_q8k(self, items: list[tuple[int, torch.Tensor, int]], workspace: torch.Tensor,
                         n_tokens: int, in_features: int, out: torch.Tensor | None = None,
                         dtype: torch.dtype = torch.float32) -> list[torch.Tensor]:
        """`matmul_multi` on activations already quantized into `workspace` (by a fused producer
        or `quantize_into`); K-quant and Q8_0 weights only. Outputs float32, or bfloat16 (`dtype`,
        or `out`'s dtype) rounded as torch's cast."""
        import ctypes

        if not 1 <= len(items) <= 4:
            raise ValueError("matmul_multi_q8k takes 1 to 4 weights")
        device = items[0][1].device
        for t, p, o in items:
            if not self.supports(t, in_features) or int(t) == 23:
                raise RuntimeError(f"mxa_gemm_multi_q8k failed with status -1 for type {t}")
            self._check_packed(int(t), p, o, in_features)
        outs = [int(o) for _, _, o in items]
        if out is None:
            out = torch.empty((n_tokens, sum(outs)), dtype=dtype, device=device)
        elif (out.dtype not in (torch.float32, torch.bfloat16) or out.device != device
              or not out.is_contiguous() or tuple(out.shape) != (n_tokens, sum(outs))):
            raise ValueError("out must be a contiguous float32 or bfloat16 (n_tokens, sum of "
                             "out_features) tensor on the weights' device")
        n = len(items)
        types = (ctypes.c_int * n)(*[int(t) for t, _, _ in items])
        ptrs = (ctypes.c_void_p * n)(*[p.data_ptr() for _, p, _ in items])
        couts = (ctypes.c_int * n)(*outs)
        fn = self._lib.mxa_gemm_multi_q8k_bf16 if out.dtype == torch.bfloat16 else \
            self._lib.mxa_gemm_multi_q8k
        status = fn(n, types, ptrs, couts, out.data_ptr(), n_tokens, in_features,
                    workspace.data_ptr(), workspace.numel(), _stream(device))
        self._check(status, "mxa_gemm_multi_q8k", int(items[0][0]))
        self._calls += 1
        return list(torch.split(out, outs, dim=-1))

    def quantize_q8_k(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Q8_K activations of x (M, K) float32 on the device: (q int8 (M, K), d float32
        (M, K/256), bsums int16 (M, K/256, 16))."""
        _require_device_tensor("x", x)
        x32 = x.detach().to(torch.float32).contiguous()
        m, k = x32.shape
        if k % 256 != 0 or m == 0:
            raise ValueError("x must be (M, K) with M > 0 and K a multiple of 256")
        nb = k // 256
        ws_bytes = q8k_bytes(m, k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        status = self._lib.mxa_quantize_q8_k(x32.data_ptr(), m, k, ws.data_ptr(), ws_bytes,
                                             _stream(x.device))
        self._check(status, "mxa_quantize_q8_k", 15)
        return q8k_views(ws, m, k)

    def dequantize(self, blocks: torch.Tensor, ggml_type: int) -> torch.Tensor:
        """`TorchDequantizer.dequantize` (app/gguf/dequant/torch_dequant.py:235-236): blocks
        (n_blocks, type_size) uint8 on the device -> (n_blocks * block_size,) float32,
        bit-exact."""
        ggml_type = int(ggml_type)
        _require_device_tensor("blocks", blocks)
        block, size = GEOMETRY[ggml_type]
        blocks = blocks.reshape(-1, size).contiguous()
        n_blocks = blocks.shape[0]
        out = torch.empty(n_blocks * block, dtype=torch.float32, device=blocks.device)
        if n_blocks == 0:
            return out
        status = self._lib.mxa_dequantize(ggml_type, blocks.data_ptr(), n_blocks, out.data_ptr(),
                                          _stream(blocks.device))
        self._check(status, "mxa_dequantize", ggml_type)
        return out

    def gather_rows(self, packed: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
        """A new (len(order), row_bytes) uint8 device tensor whose row i is `packed` row
        `order[i]` (`PackedRows.reordered`, app/gguf/packed_rows.py:24-28, on the device).
        Indices are checked on the host: an index outside [0, n_rows) raises IndexError."""
        _require_device_tensor("packed", packed)
        if packed.dtype != torch.uint8 or packed.dim() != 2 or not packed.is_contiguous():
            raise ValueError("packed must be a contiguous uint8 (n_rows, row_bytes) tensor")
        idx = order.detach().reshape(-1).to(torch.int64)
        n = idx.numel()
        out = torch.empty((n, packed.shape[1]), dtype=torch.uint8, device=packed.device)
        if n == 0:
            return out
        lo, hi = int(idx.min()), int(idx.max())
        if lo < 0 or hi >= packed.shape[0]:
            raise IndexError(f"row index out of range [0, {packed.shape[0]}): {lo if lo < 0 else hi}")
        idx32 = idx.to(device=packed.device, dtype=torch.int32)
        status = self._lib.mxa_gather_rows(packed.data_ptr(), packed.shape[0], packed.shape[1],
                                           idx32.data_ptr(), n, out.data_ptr(),
                                           _stream(packed.device))
        self._check(status, "mxa_gather_rows", 0)
        return out

    def stream_read(self, data: torch.Tensor, sink: torch.Tensor) -> None:
        """Measurement aid (no reference counterpart): one launch that reads every byte of the
        contiguous device tensor `data` once and computes nothing from them; `sink` is a device
        int32 word it may write. Its time is the floor of a one-launch kernel over those bytes."""
        _require_device_tensor("data", data)
        _require_device_tensor("sink", sink)
        nbytes = data.numel() * data.element_size()
        if not data.is_contiguous() or nbytes % 16 or data.data_ptr() % 16:
            raise ValueError("data must be contiguous, 16-byte aligned, a multiple of 16 bytes")
        status = self._lib.mxa_stream_read(data.data_ptr(), nbytes, sink.data_ptr(),
                                           _stream(data.device))
        self._check(status, "mxa_stream_read", 0)

    def dequant_rows(self, ggml_type: int, packed: torch.Tensor, row_indices: torch.Tensor,
                     row_width: int) -> torch.Tensor:
        """Rows `row_indices` of the packed (n_rows, row_bytes) matrix, dequantized bit-exactly
        to (len(row_indices), row_width) float32 (NativeGemm.dequant_rows,
        app/native/gemm.py:111-132, on the device). An index outside [0, n_rows), also one past
        the int32 range, gives a row of NaN: the kernel never reads outside the table, and the
        call never waits for the host to check."""
        ggml_type = int(ggml_type)
        if not self.supports_dequant_rows(ggml_type, row_width):
            raise RuntimeError(f"mxa_dequant_rows failed with status -1 for type {ggml_type}")
        self._check_packed(ggml_type, packed, packed.shape[0], row_width)
        n_rows = packed.shape[0]
        idx = row_indices.detach().reshape(-1).to(device=packed.device, dtype=torch.int64)
        idx = idx.clamp(-1, n_rows).to(torch.int32).contiguous()
        out = torch.empty((idx.shape[0], row_width), dtype=torch.float32, device=packed.device)
        if idx.shape[0] == 0:
            return out
        status = self._lib.mxa_dequant_rows(ggml_type, packed.data_ptr(), packed.shape[0],
                                            idx.data_ptr(), idx.shape[0], row_width,
                                            out.data_ptr(), _stream(packed.device))
        self._check(status, "mxa_dequant_rows", ggml_type)
        return out
