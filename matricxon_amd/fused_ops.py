"""Device twins of the reference's fused producer ops and shared-input projections, for packed
weights on the GPU:

* `HipFusedOps.rms_norm(x, weight, eps)` / `.silu_mul(gate, up)`: the `FusedOps` methods that
  `RMSNorm.forward` and `SwiGLUMLP.forward` call (app/native/fused_ops.py:152-158, 201-208;
  app/architectures/layers.py:53-57, 72-76), same contract: the result, or None when the inputs
  are not handled (not all float32 or all bfloat16 on a GPU, mismatched shapes, a last dimension
  that is not a multiple of 256) so the caller runs its torch code. Float32 inputs get the
  reference C kernels' float32 steps (mx_fused_ops.c); bfloat16 inputs, the dtype of the
  reference's GPU layers (app/runtime/compute_device.py:74-78), get the steps of the torch code the
  reference runs for them (layers.py:53-57, 77-81), each elementwise result rounded to bfloat16
  where torch rounds it. Each also writes the Q8_K blocks of its result in the same kernel and
  hands them to the packed projections that read that result.
* `project_shared(owner, names, x)`: `owner.<name>(x)` for each name, as one
  `mxa_gemm_multi` call when every module is a `DevicePackedLinear` over the same input (the
  device side of app/architectures/shared_projection.py:33-43).

The hand-off keeps, per host thread, the most recent producer result and its Q8_K blocks. A
projection takes them only when its input is that very result: the same storage, element count
and dtype, unmodified since (a tensor's version counter, shared by its views, moves on any in-place
write), on the device and stream the producer ran on. Holding the result keeps its memory from
being reused by another tensor while the blocks are offered.
"""

import threading

import torch
from torch import nn

from matricxon_amd.gemm import HipGemm

_IQ4_XS = 23


def _stream_of(device: torch.device) -> int | None:
    return torch.cuda.current_stream(device).cuda_stream if device.type == "cuda" else None


class _Handoff:
    """The calling thread's last producer result and the workspace holding its Q8_K blocks.

    One slot per host thread: the reference runs one worker thread per loaded model
    (app/models/worker.py:15-46), so two models' forwards can interleave, and a thread must only
    ever claim blocks it offered itself. The slot is one tuple, replaced whole, so a claim never
    sees the parts of two different offers.
    """

    def __init__(self) -> None:
        self._local = threading.local()

    def offer(self, out: torch.Tensor, workspace: torch.Tensor) -> None:
        self._local.slot = (out, out._version, workspace, out.device, _stream_of(out.device))

    def clear(self) -> None:
        """Drops the calling thread's offer."""
        self._local.slot = None

    def claim(self, x: torch.Tensor) -> torch.Tensor | None:
        """The Q8_K workspace of x if x is this thread's offered result, unchanged, on the stream
        it was produced on; else None."""
        slot = getattr(self._local, "slot", None)
        if slot is None or not x.is_contiguous():
            return None
        out, version, workspace, device, stream = slot
        if (x.dtype != out.dtype or x.device != device or x.data_ptr() != out.data_ptr()
                or x.numel() != out.numel()
                or x.shape[-1] != out.shape[-1] or x._version != version
                or out._version != version or _stream_of(device) != stream):
            return None
        return workspace


HANDOFF = _Handoff()


_RMS_BF16_MAX = 16384  # the bfloat16 RMSNorm kernel's longest row


def _handled(*tensors: torch.Tensor) -> bool:
    """All on a GPU and all float32, or all bfloat16."""
    dt = tensors[0].dtype
    return dt in (torch.float32, torch.bfloat16) and all(
        t.dtype == dt and t.device.type == "cuda" for t in tensors)


class HipFusedOps:
    """`FusedOps` (app/native/fused_ops.py:128-150) for GPU tensors: `configure` / `active`
    select it, and each method returns None for inputs it does not handle."""

    _active: "HipFusedOps | None" = None

    def __init__(self) -> None:
        self._gemm = HipGemm.get()

    @classmethod
    def configure(cls, enabled: bool) -> None:
        HANDOFF.clear()
        cls._active = cls() if enabled else None

    @classmethod
    def active(cls) -> "HipFusedOps | None":
        return cls._active

    def rms_norm(self, x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor | None:
        """x * (1 / sqrt(mean(x^2) + eps)) * weight over the last dimension (layers.py:72-81)."""
        if (not _handled(x, weight) or weight.dim() != 1 or x.shape[-1] != weight.shape[0]
                or x.shape[-1] % 256 != 0 or x.numel() == 0
                or (x.dtype == torch.bfloat16 and x.shape[-1] > _RMS_BF16_MAX)):
            return None
        out, ws = self._gemm.rms_norm_q8k(x, weight, eps)
        out = out.view(x.shape)
        HANDOFF.offer(out, ws)
        return out

    def silu_mul(self, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor | None:
        """silu(gate) * up elementwise (layers.py:53-57)."""
        if (not _handled(gate, up) or gate.shape != up.shape or gate.dim() == 0
                or gate.shape[-1] % 256 != 0 or gate.numel() == 0):
            return None
        out, ws = self._gemm.silu_mul_q8k(gate, up)
        out = out.view(gate.shape)
        HANDOFF.offer(out, ws)
        return out


def project_shared(owner: nn.Module, names: tuple[str, ...], x: torch.Tensor) -> list[torch.Tensor]:
    """`owner.<name>(x)` for each name: one launch group for up to 4 `DevicePackedLinear` modules
    of one input width and dtype, else each module on its own (shared_projection.py:33-43)."""
    from matricxon_amd.device_packed import DevicePackedLinear

    mods = [getattr(owner, name) for name in names]
    if (not 1 <= len(mods) <= 4 or x.device.type != "cuda"
            or not all(isinstance(m, DevicePackedLinear) for m in mods)
            or len({m.in_features for m in mods}) != 1 or len({m.dtype for m in mods}) != 1
            or len({m.packed.device for m in mods}) != 1 or x.shape[-1] != mods[0].in_features):
        return [m(x) for m in mods]
    dtype, k = mods[0].dtype, mods[0].in_features
    lead = x.shape[:-1]
    xd = x.to(dtype)  # each module casts x to its dtype first (device_packed.py:54)
    items = [(m.ggml_type, m.packed, m.out_features) for m in mods]
    gemm = HipGemm.get()
    bf16 = dtype == torch.bfloat16  # bfloat16 outputs straight from the kernels
    ws = HANDOFF.claim(xd)
    if ws is not None and all(t != _IQ4_XS for t, _, _ in items):
        ys = gemm.matmul_multi_q8k(items, ws, xd.numel() // k, k,
                                   dtype=torch.bfloat16 if bf16 else torch.float32)
    else:
        ys = gemm.matmul_multi(items, xd.reshape(-1, k), bf16=bf16)
    return [m.finish(y, lead) for m, y in zip(mods, ys, strict=True)]
