"""Several packed device weights that share one input (q/k/v, gate/up) as one library call
(`mxa_gemm_multi`): the input is quantized once and, for up to 16 tokens, every weight's rows run
in one launch.

`MultiGemmPlan` mirrors the reference's plan of the same name (app/native/gemm_multi.py:15-61):
`build(items, in_features)` once per group, returning None when the library is not configured or a
weight has no kernel; `run(x)` per call, returning one float32 output per weight, or None when the
library declines the call (status -1) so the caller runs each weight on its own. The weights are
device uint8 tensors of packed rows instead of mmap'd memoryviews, and the call is asynchronous on
torch's current stream.
"""

import ctypes

import torch

from matricxon_amd.gemm import HipGemm, _stream

_IQ4_XS = 23


class MultiGemmPlan:
    def __init__(self, gemm: HipGemm, types: list[int], packed: list[torch.Tensor],
                 outs: list[int], in_features: int) -> None:
        self._gemm = gemm
        self._fn = gemm._lib.mxa_gemm_multi
        self._n = len(types)
        self._types = (ctypes.c_int * self._n)(*types)
        self._ptrs = (ctypes.c_void_p * self._n)(*[p.data_ptr() for p in packed])
        self._outs = (ctypes.c_int * self._n)(*outs)
        self._packed = packed  # keeps the weights alive while the plan holds their addresses
        self._kinds = {int(t) == _IQ4_XS for t in types}
        self.device = packed[0].device
        self.outs = list(outs)
        self.in_features = in_features
        self._total = sum(outs)

    @classmethod
    def build(cls, items: list[tuple[int, torch.Tensor, int]],
              in_features: int) -> "MultiGemmPlan | None":
        """`items`: (ggml_type, packed, out_features) per weight, `packed` a contiguous device
        uint8 (out_features, row_bytes) tensor. None without a configured library, for fewer
        than 2 or more than 4 weights, weights on different devices, or any weight without a
        kernel (app/native/gemm_multi.py:29-44)."""
        gemm = HipGemm.active()
        if gemm is None or not 1 < len(items) <= 4:
            return None
        if not all(gemm.supports(t, in_features) for t, _, _ in items):
            return None
        devices = {p.device for _, p, _ in items}
        if len(devices) != 1 or next(iter(devices)).type != "cuda":
            return None
        for t, p, o in items:
            gemm._check_packed(int(t), p, int(o), in_features)
        return cls(gemm, [int(t) for t, _, _ in items], [p for _, p, _ in items],
                   [int(o) for _, _, o in items], in_features)

    def workspace_bytes(self, n_tokens: int) -> int:
        """Workspace of one call over n_tokens rows: the Q8_K part and, with an IQ4_XS weight,
        the split part after it."""
        need = 0
        for is_iq4 in self._kinds:
            need += self._gemm.workspace_bytes(_IQ4_XS if is_iq4 else 12, n_tokens,
                                               self.in_features)
        return need

    def run(self, x: torch.Tensor) -> list[torch.Tensor] | None:
        """`x` (n_tokens, in_features): one float32 output per weight, (n_tokens, out_i), views of
        one (n_tokens, sum of outs) buffer; None when the library declines the call (the caller
        then runs each weight, app/native/gemm_multi.py:46-61)."""
        x32 = x.detach().reshape(-1, self.in_features).to(device=self.device,
                                                          dtype=torch.float32).contiguous()
        n_tokens = x32.shape[0]
        y = torch.empty((n_tokens, self._total), dtype=torch.float32, device=self.device)
        if n_tokens == 0:
            return list(torch.split(y, self.outs, dim=-1))
        ws_bytes = self.workspace_bytes(n_tokens)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=self.device)
        status = self._fn(self._n, self._types, self._ptrs, self._outs, x32.data_ptr(),
                          y.data_ptr(), n_tokens, self.in_features, ws.data_ptr(), ws_bytes,
                          _stream(self.device))
        if status == -1:
            return None
        self._gemm.record()
        self._gemm._check(status, "mxa_gemm_multi", int(self._types[0]))
        return list(torch.split(y, self.outs, dim=-1))
