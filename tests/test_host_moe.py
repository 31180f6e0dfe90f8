"""Host logic of the grouped MoE experts on the CPU: the device-side routing table
(`route_pairs`) and the per-token combine (`combine_in_expert_order`) against the reference's own
loop (app/architectures/moe_experts.py:81-88) on random contributions, bit for bit."""

import torch

from matricxon_amd.moe import combine_in_expert_order, route_pairs


def test_route_pairs_groups_pairs_by_expert() -> None:
    idx = torch.tensor([[3, 0], [1, 3], [0, 2], [3, 1]])
    order, offsets, pair_tok = route_pairs(idx, 5)
    assert offsets.dtype == torch.int32
    assert offsets.tolist() == [0, 2, 4, 5, 8, 8]  # expert 4 has no pair
    assert order.tolist() == [1, 4, 2, 7, 5, 0, 3, 6]  # tokens ascending within an expert
    assert pair_tok.tolist() == [0, 2, 1, 3, 2, 0, 1, 3]
    flat = idx.reshape(-1)
    for e in range(5):
        assert (flat[order[offsets[e]:offsets[e + 1]]] == e).all()


def test_route_pairs_clamps_bad_ids() -> None:
    _, offsets, _ = route_pairs(torch.tensor([[-1, 9]]), 4)
    assert offsets.tolist() == [0, 1, 1, 1, 2]


def reference_combine(per_pair: torch.Tensor, top_k_idx: torch.Tensor) -> torch.Tensor:
    """moe_experts.py:81-88 with the expert work replaced by `per_pair` (n_tokens, top_k, d)."""
    n_tokens, _ = top_k_idx.shape
    out = torch.zeros(n_tokens, per_pair.shape[-1], dtype=torch.float32)
    for expert_id in top_k_idx.unique().tolist():
        token_idx, k_idx = (top_k_idx == expert_id).nonzero(as_tuple=True)
        out.index_add_(0, token_idx, per_pair[token_idx, k_idx].to(torch.float32))
    return out


def test_combine_adds_in_ascending_expert_order() -> None:
    g = torch.Generator().manual_seed(0)
    for n_tokens, n_experts, top_k in ((1, 4, 1), (13, 8, 2), (64, 32, 4), (7, 5, 5)):
        idx = torch.stack([torch.randperm(n_experts, generator=g)[:top_k]
                           for _ in range(n_tokens)])
        # magnitudes spread over many binades so that another summation order rounds otherwise
        per_pair = torch.randn(n_tokens, top_k, 96, generator=g) * \
            torch.exp2(torch.randint(-20, 20, (n_tokens, top_k, 96), generator=g).float())
        order, _, _ = route_pairs(idx, n_experts)
        contrib = per_pair.reshape(-1, 96).index_select(0, order)
        got = combine_in_expert_order(contrib, order, idx)
        want = reference_combine(per_pair, idx)
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_fused_combine_gate() -> None:
    # the one-launch combine takes float32 weights, float32 / bfloat16 layers, at most 16 slots
    # and 65535 tokens; anything else keeps the torch steps
    import torch
    from matricxon_amd.moe import HipPackedMoEExperts

    mod = HipPackedMoEExperts.__new__(HipPackedMoEExperts)
    mod.dtype = torch.bfloat16
    assert mod._fused_combine(torch.zeros(4, 2))
    assert not mod._fused_combine(torch.zeros(4, 2, dtype=torch.bfloat16))
    assert not mod._fused_combine(torch.zeros(4, 17))
    assert not mod._fused_combine(torch.zeros(65536, 2))
    mod.dtype = torch.float16
    assert not mod._fused_combine(torch.zeros(4, 2))
