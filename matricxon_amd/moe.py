"""Packed MoE experts on the device with one grouped launch per projection: the drop-in for the
reference's `QuantizedMoEExperts` in packed-GPU mode (app/architectures/moe_experts.py:29-89).

The reference loops over the routed experts on the host (`top_k_idx.unique().tolist()`, a host
sync), gathers each expert's tokens and calls that expert's `DevicePackedLinear` three times, then
adds each expert's weighted output into the result in ascending expert order (moe_experts.py:81-88).
Here the routing is sorted on the device into (token, expert) pairs grouped by expert, and each
projection is one `mxa_gemm_moe` launch over all experts. Every pair row equals the reference's
per-expert row bit for bit (the same packed matmul per row), the projections' outputs take the
module's dtype as the reference's modules return it, and the weighted outputs are added per token
in ascending expert order, so the result is the reference's bit for bit.
"""

from collections.abc import Callable

import torch
from torch import nn

from .gemm import HipGemm, q8k_bytes


def route_pairs(top_k_idx: torch.Tensor, num_experts: int) -> tuple[torch.Tensor, torch.Tensor,
                                                                    torch.Tensor]:
    """(order, offsets, pair_tok) of the routing (n_tokens, top_k), all on its device and without
    a host sync: `order` sorts the flattened (token, slot) pairs by expert (stable: tokens
    ascending within an expert), `offsets` (num_experts + 1, int32) delimits each expert's pairs,
    and `pair_tok` is the token of each sorted pair. Expert ids outside [0, num_experts) are
    clamped into it (a router never produces them; clamping keeps a bad id from indexing past
    the counts)."""
    flat = top_k_idx.reshape(-1).to(torch.int64).clamp(0, num_experts - 1)
    order = torch.argsort(flat, stable=True)
    counts = torch.zeros(num_experts, dtype=torch.int64, device=flat.device)
    counts.scatter_add_(0, flat, torch.ones_like(flat))
    offsets = torch.zeros(num_experts + 1, dtype=torch.int32, device=flat.device)
    offsets[1:] = torch.cumsum(counts, 0).to(torch.int32)
    pair_tok = order // top_k_idx.shape[1]
    return order, offsets, pair_tok


def combine_in_expert_order(contrib: torch.Tensor, order: torch.Tensor, top_k_idx: torch.Tensor
                            ) -> torch.Tensor:
    """out[t] = the float32 contributions of token t's pairs added in ascending expert order, as
    the reference's loop of `index_add_` over the sorted expert ids adds them
    (app/architectures/moe_experts.py:81-88). `contrib` (n_pairs, n_embd) float32 is in the
    expert-sorted pair order `order`."""
    n_tokens, top_k = top_k_idx.shape
    by_pair = torch.empty_like(contrib)
    by_pair.index_copy_(0, order, contrib)  # back to (token, slot) order
    slot_order = torch.argsort(top_k_idx, dim=1, stable=True)
    rows = torch.arange(n_tokens, device=contrib.device).unsqueeze(1) * top_k + slot_order
    out = torch.zeros(n_tokens, contrib.shape[1], dtype=torch.float32, device=contrib.device)
    for r in range(top_k):
        out += by_pair.index_select(0, rows[:, r])
    return out


_IQ4_XS = 23  # float activations: no Q8_K blocks


def _is_silu(fn) -> bool:
    """Whether the experts' activation is SiLU (the fused producer computes exactly its steps)."""
    return fn is torch.nn.functional.silu or isinstance(fn, torch.nn.SiLU)


class HipPackedMoEExperts(nn.Module):
    """Packed expert FFN: gate/up/down as (num_experts, out_features, row_bytes) packed bytes on
    the device (`matricxon_amd.loading.PackedUploader.upload_experts`), all of one GGUF type each.
    `forward(x, top_k_weights, top_k_idx)` has the reference's signature and result."""

    def __init__(self, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor,
                 gate_type: int, up_type: int, down_type: int, n_embd: int, ffn_len: int,
                 activation: Callable[[torch.Tensor], torch.Tensor],
                 dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.num_experts = gate.shape[0]
        self.n_embd, self.ffn_len = n_embd, ffn_len
        self.activation = activation
        self.dtype = dtype
        self.types = (int(gate_type), int(up_type), int(down_type))
        self._gemm = HipGemm.get()
        for t, k in ((gate_type, n_embd), (up_type, n_embd), (down_type, ffn_len)):
            if not self._gemm.supports(int(t), k):
                raise ValueError(f"no grouped HIP projection for GGUF type {int(t)}")
        for name, w in (("gate", gate), ("up", up), ("down", down)):
            if w.dim() != 3 or w.shape[0] != self.num_experts or (w.shape[1] * w.shape[2]) % 4:
                raise ValueError(f"{name} experts must be (num_experts, out, row_bytes) with each "
                                 "expert's bytes a multiple of 4")
        # the one-token pairs launch takes K / 256 in {4, 8, 16, 32, 56, 64} and 16-byte aligned
        # rows; other shapes go straight to the grouped launch
        # (K-quant and Q8_0 experts; IQ4_XS experts take the grouped launch)
        self._pairs = all(int(t) != 23 and k // 256 in (4, 8, 16, 32, 56, 64) and
                          self._gemm.row_bytes(int(t), k) % 16 == 0
                          for t, k in ((gate_type, n_embd), (up_type, n_embd), (down_type, ffn_len)))
        self.register_buffer("gate_packed", gate, persistent=False)
        self.register_buffer("up_packed", up, persistent=False)
        self.register_buffer("down_packed", down, persistent=False)

    def forward(self, x: torch.Tensor, top_k_weights: torch.Tensor,
                top_k_idx: torch.Tensor) -> torch.Tensor:
        n_tokens, n_embd = x.shape
        top_k = top_k_idx.shape[1]
        if n_tokens == 1 and self._pairs:
            out = self._one_token(x, top_k_weights, top_k_idx)
            if out is not None:
                return out
        g = self._gemm
        fused = self._fused_combine(top_k_weights)
        if fused and self.num_experts <= g.MOE_ROUTE_MAX_EXPERTS and \
                0 < n_tokens * top_k <= g.MOE_ROUTE_MAX_PAIRS and \
                top_k_idx.dtype in (torch.int32, torch.int64):
            # one launch: the sort, each pair's token and place, the ids as int32 for the combine
            order = None
            offsets, pair_tok, rows, ids32 = g.moe_route(top_k_idx, self.num_experts)
        else:
            order, offsets, pair_tok = route_pairs(top_k_idx, self.num_experts)
        # the reference casts x to the layer dtype before each matmul (device_packed.py:54)
        xs = x.to(self.dtype).index_select(0, pair_tok)  # each pair's token, by expert
        # the launch is sized for one row per token and expert; an expert that a token's routing
        # names twice (the reference computes both slots) gets its extra rows by the kernel's loop
        bound = n_tokens
        gt, ut, dt = self.types
        n_pairs, dev = xs.shape[0], x.device
        # a bfloat16 layer's projections return bfloat16 (device_packed.py:53-58): the launches
        # write gate and up rounded as that cast rounds them
        gu = torch.bfloat16 if self.dtype == torch.bfloat16 else torch.float32
        if n_pairs > 0 and _IQ4_XS not in (gt, ut) and xs.dtype in (torch.float32, torch.bfloat16):
            # gate and up share one Q8_K quantization of the pairs' rows (the same blocks each
            # call would write: bfloat16 values are widened exactly first)
            wsx = torch.empty(q8k_bytes(n_pairs, n_embd), dtype=torch.uint8, device=dev)
            g.quantize_into(xs, wsx)
            gate = g.matmul_moe(gt, self.gate_packed, None, offsets, bound, self.ffn_len, n_embd,
                                workspace=wsx, out=torch.empty((n_pairs, self.ffn_len),
                                                               dtype=gu, device=dev),
                                out_dtype=gu)
            up = g.matmul_moe(ut, self.up_packed, None, offsets, bound, self.ffn_len, n_embd,
                              workspace=wsx, out=torch.empty((n_pairs, self.ffn_len),
                                                             dtype=gu, device=dev),
                              out_dtype=gu)
        else:
            gate = g.matmul_moe(gt, self.gate_packed, xs, offsets, bound, self.ffn_len, n_embd,
                                out_dtype=gu)
            up = g.matmul_moe(ut, self.up_packed, xs, offsets, bound, self.ffn_len, n_embd,
                              out_dtype=gu)
        if n_pairs > 0 and dt != _IQ4_XS and self.dtype == torch.bfloat16 and \
                _is_silu(self.activation):
            # F.silu(gate) * up with torch's bfloat16 steps and the down projection's Q8_K blocks of
            # exactly that tensor in one launch (as the one-token path does)
            _, wsa = g.silu_mul_q8k(gate.to(self.dtype), up.to(self.dtype), want_out=False)
            down = g.matmul_moe(dt, self.down_packed, None, offsets, bound, n_embd, self.ffn_len,
                                workspace=wsa, out=torch.empty((n_pairs, n_embd),
                                                               dtype=torch.float32, device=dev))
        else:
            act = self.activation(gate.to(self.dtype)) * up.to(self.dtype)
            down = g.matmul_moe(dt, self.down_packed, act, offsets, bound, n_embd, self.ffn_len)
        if order is None:
            return self._combine(down, rows, ids32, top_k_weights).to(x.dtype)
        if fused:
            # down row of pair p = its place in the sorted order
            rows = torch.empty_like(order)
            rows[order] = torch.arange(order.numel(), device=order.device)
            return self._combine(down, rows, top_k_idx, top_k_weights).to(x.dtype)
        w = top_k_weights.reshape(-1).index_select(0, order).unsqueeze(-1)
        contrib = (down.to(self.dtype) * w).to(torch.float32)  # sorted pair order
        return combine_in_expert_order(contrib, order, top_k_idx).to(x.dtype)

    def _fused_combine(self, top_k_weights: torch.Tensor) -> bool:
        """Whether the weighted combine runs as one `mxa_moe_combine` launch: float32 routing
        weights, a float32 or bfloat16 layer dtype, at most 16 experts per token and 65535 tokens
        (the launch's grid)."""
        return (top_k_weights.dtype == torch.float32 and top_k_weights.shape[-1] <= 16
                and top_k_weights.shape[0] <= 65535
                and self.dtype in (torch.float32, torch.bfloat16))

    def _combine(self, down: torch.Tensor, rows: torch.Tensor | None, top_k_idx: torch.Tensor,
                 top_k_weights: torch.Tensor) -> torch.Tensor:
        """float32 (n_tokens, n_embd): the reference's `down.to(dtype) * weight` contributions
        `index_add_`ed in ascending expert order, in one launch."""
        shape = top_k_idx.shape
        ids = top_k_idx if top_k_idx.dtype == torch.int32 else top_k_idx.to(torch.int32)
        ids = ids.contiguous()
        if rows is not None:
            rows = rows.to(torch.int32).reshape(shape).contiguous()
        return self._gemm.moe_combine(down, ids, top_k_weights.contiguous(), rows,
                                      round_bf16=self.dtype == torch.bfloat16)

    def _one_token(self, x: torch.Tensor, top_k_weights: torch.Tensor,
                   top_k_idx: torch.Tensor) -> torch.Tensor | None:
        """Decode: each routed expert is a distinct pair of the one token, so the projections
        run as pairs (`mxa_gemm_moe_pairs`, expert ids read on the device) without sorting the
        routing. None when a projection's shape does not suit that launch."""
        g = self._gemm
        gt, ut, dt = self.types
        ids = top_k_idx.to(torch.int32).contiguous()
        if self.dtype == torch.bfloat16 and _is_silu(self.activation):
            out = self._one_token_bf16(x, top_k_weights, ids)
            if out is not None:
                return out
        # the reference casts x to the layer dtype before each matmul (device_packed.py:54); the
        # kernels take float32, so the cast values are widened once for both projections
        xs = x.to(self.dtype).to(torch.float32)
        gate = g.matmul_moe_pairs(gt, self.gate_packed, ids.view(-1), xs, self.ffn_len, self.n_embd)
        if gate is None:
            return None
        up = g.matmul_moe_pairs(ut, self.up_packed, ids.view(-1), xs, self.ffn_len, self.n_embd)
        if up is None:
            return None
        act = self.activation(gate.to(self.dtype)) * up.to(self.dtype)
        down = g.matmul_moe_pairs(dt, self.down_packed, ids.view(-1), act, self.n_embd, self.ffn_len)
        if down is None:
            return None
        if self._fused_combine(top_k_weights):
            return self._combine(down, None, ids, top_k_weights).to(x.dtype)
        w = top_k_weights.reshape(-1).unsqueeze(-1)
        contrib = (down.to(self.dtype) * w).to(torch.float32)  # slot order
        slot = torch.arange(ids.numel(), device=x.device)
        return combine_in_expert_order(contrib, slot, top_k_idx).to(x.dtype)

    def _one_token_bf16(self, x: torch.Tensor, top_k_weights: torch.Tensor,
                        ids: torch.Tensor) -> torch.Tensor | None:
        """The one-token forward of a bfloat16 layer with a SiLU activation in four library
        launches and no casts: gate and up read the bfloat16 x and write bfloat16 (the reference's
        `gate.to(dtype)`, `up.to(dtype)`), the fused producer computes `F.silu(gate) * up` with
        torch's bfloat16 steps and writes the down projection's Q8_K blocks of exactly that tensor,
        and the down projection runs on them; then the combine. The same bits as the unfused steps
        (moe_experts.py:81-88 through device_packed.py:53-63). None when a launch does not take
        the shapes (the caller runs the float32 steps)."""
        g = self._gemm
        gt, ut, dt = self.types
        idv = ids.view(-1)
        if not self._fused_combine(top_k_weights):
            return None
        xb = x.to(torch.bfloat16)
        gate = g.matmul_moe_pairs(gt, self.gate_packed, idv, xb, self.ffn_len, self.n_embd,
                                  out_dtype=torch.bfloat16)
        if gate is None:
            return None
        up = g.matmul_moe_pairs(ut, self.up_packed, idv, xb, self.ffn_len, self.n_embd,
                                out_dtype=torch.bfloat16)
        if up is None:
            return None
        _, ws = g.silu_mul_q8k(gate, up, want_out=False)
        down = g.matmul_moe_pairs(dt, self.down_packed, idv, None, self.n_embd, self.ffn_len,
                                  workspace=ws, x_rows=idv.numel())
        if down is None:
            return None
        return self._combine(down, None, ids, top_k_weights).to(x.dtype)

    @classmethod
    def from_packed_bytes(cls, gate_raw, up_raw, down_raw, types: tuple[int, int, int],
                          num_experts: int, n_embd: int, ffn_len: int,
                          activation: Callable[[torch.Tensor], torch.Tensor],
                          dtype: torch.dtype, device: torch.device) -> "HipPackedMoEExperts":
        """From the GGUF bytes of the three expert tensors ((num_experts, out, in) each, as
        `loader.raw_tensor_bytes_and_type` returns them for moe_experts.py:108-121), uploaded
        still packed, one allocation per tensor."""
        from .loading import PackedUploader

        with PackedUploader(device) as up:
            gate, _ = up.upload_experts(gate_raw, num_experts, ffn_len)
            upw, _ = up.upload_experts(up_raw, num_experts, ffn_len)
            down, _ = up.upload_experts(down_raw, num_experts, n_embd)
        return cls(gate, upw, down, *types, n_embd, ffn_len, activation, dtype)
