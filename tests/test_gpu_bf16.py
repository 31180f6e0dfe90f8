"""bfloat16 layers on the GPU, the reference's GPU dtype (app/runtime/compute_device.py:74-78):
the matmul entry points that read bfloat16 x and write bfloat16 y (`mxa_gemm_bf16`,
`mxa_gemm_multi_bf16`, `mxa_gemm_q8k_bf16`, `mxa_gemm_multi_q8k_bf16`), the bfloat16 fused
producers (`mxa_rms_norm_q8_k_bf16`, `mxa_silu_mul_q8_k_bf16`) and a bfloat16 layer through the
hand-off.

Bars: a bfloat16 output equals, bit for bit, the float32 entry point's output on the widened x
rounded by torch's own float -> bfloat16 cast (which the oracle's float32 result pins in turn);
the producers' Q8_K blocks equal those of quantizing their bfloat16 result; silu * up equals
torch's `F.silu(gate) * up` on bfloat16 tensors bit for bit; RMSNorm is within one bfloat16 ulp
of torch's steps (its sum of squares and rsqrt are reduced and rounded in another order)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as TF
from torch import nn

from matricxon_amd import synthetic as S
from matricxon_amd.device_packed import DevicePackedLinear
from matricxon_amd.fused_ops import HANDOFF, HipFusedOps, project_shared
from matricxon_amd.gemm import q8k_views
from oracle import dequant as D
from tests.test_gpu_kernels import dev, host

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def bf16_bits(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().view(torch.int16)


def x_bf16(m: int, k: int, seed: int) -> torch.Tensor:
    return dev(S.activations(m, k, seed=seed)).to(BF)


# (type, N, K, M): one-row floor-shaped kernel (bf16 x read by the kernel), its two / three-row
# forms, shapes it does not take (x quantized into the workspace first), batched decode, prefill
CASES = [
    (D.Q4_K, 4096, 4096, 1), (D.Q4_K, 14336, 4096, 1), (D.Q6_K, 1024, 4096, 1),
    (D.Q8_0, 512, 4096, 1), (D.Q4_K, 4096, 14336, 1), (D.Q6_K, 300, 14336, 1),
    (D.Q4_K, 2048, 4096, 2), (D.Q6_K, 1024, 2048, 3), (D.Q4_K, 700, 768, 1),
    (D.Q4_K, 512, 2304, 2), (D.Q6_K, 4096, 4096, 4), (D.Q4_K, 4096, 4096, 16),
    (D.Q8_0, 1000, 2048, 9), (D.Q4_K, 1024, 4096, 64), (D.IQ4_XS, 1024, 4096, 1),
    (D.IQ4_XS, 512, 2048, 7), (D.IQ4_XS, 256, 4096, 20),
]


@pytest.mark.parametrize("t,n,k,m", CASES)
def test_gemm_bf16_is_the_float32_result_rounded(gpu, oracle, t, n, k, m) -> None:
    w_np = S.packed_weight(t, n, k, seed=n + m)
    w = dev(w_np)
    xb = x_bf16(m, k, seed=k + m)
    got = gpu.matmul_bf16(t, w, xb, n, k)
    assert got.dtype == BF and got.shape == (m, n)
    y32 = gpu.matmul(t, w, xb.to(torch.float32), n, k)
    assert torch.equal(bf16_bits(got), bf16_bits(y32.to(BF)))
    if t != D.IQ4_XS:  # K-quants: the oracle's float32 bits, rounded on the CPU by torch's cast
        want = torch.from_numpy(oracle.gemm(t, w_np, host(xb.to(torch.float32)), n, k)).to(BF)
        assert torch.equal(bf16_bits(got), want.view(torch.int16))


def test_bf16_rounding_of_special_outputs(gpu) -> None:
    """Zero weight rows, huge and tiny outputs: ties to even and the exponent range of the cast."""
    t, n, k = D.Q8_0, 256, 2048
    w_np = S.packed_weight(t, n, k, seed=3)
    w_np[:8] = 0  # rows of zeros: +0
    scale = np.frombuffer(np.float16(60000.0).tobytes(), dtype=np.uint8)
    blocks = w_np[8:16].reshape(8, -1, 34)
    blocks[:, :, 0:2] = scale  # large d: outputs near the float32 range of the cast
    w = dev(w_np)
    xb = (x_bf16(1, k, seed=4) * 1000).to(BF)
    got = gpu.matmul_bf16(t, w, xb, n, k)
    y32 = gpu.matmul(t, w, xb.to(torch.float32), n, k)
    assert torch.equal(bf16_bits(got), bf16_bits(y32.to(BF)))


@pytest.mark.parametrize("m", [1, 3, 16, 40])
def test_gemm_multi_bf16(gpu, m) -> None:
    k = 4096
    items = [(D.Q4_K, dev(S.packed_weight(D.Q4_K, 1024, k, seed=1)), 1024),
             (D.Q4_K, dev(S.packed_weight(D.Q4_K, 256, k, seed=2)), 256),
             (D.Q6_K, dev(S.packed_weight(D.Q6_K, 256, k, seed=3)), 256)]
    xb = x_bf16(m, k, seed=m)
    ys = gpu.matmul_multi(items, xb, bf16=True)
    for (t, w, n), y in zip(items, ys):
        assert y.dtype == BF
        want = gpu.matmul(t, w, xb.to(torch.float32), n, k).to(BF)
        assert torch.equal(bf16_bits(y), bf16_bits(want))


@pytest.mark.parametrize("m,k", [(1, 4096), (16, 4096), (5, 14336)])
def test_quantize_bf16_equals_quantize_of_widened(gpu, m, k) -> None:
    xb = x_bf16(m, k, seed=7)
    xb[0, :256] = 0  # an all-zero block
    ws = torch.empty(200_000 * m, dtype=torch.uint8, device="cuda")
    gpu.quantize_into(xb, ws)
    for a, b in zip(q8k_views(ws, m, k), gpu.quantize_q8_k(xb.to(torch.float32))):
        assert torch.equal(a, b)


def assert_q8k_of(gpu, ws: torch.Tensor, out: torch.Tensor) -> None:
    m, k = out.shape
    for name, g, w in zip(("q", "d", "bsums"), q8k_views(ws, m, k),
                          gpu.quantize_q8_k(out.to(torch.float32))):
        assert torch.equal(g, w), name


@pytest.mark.parametrize("m,k", [(1, 4096), (3, 4096), (16, 4096), (2, 14336), (7, 256)])
def test_rms_norm_bf16_follows_torch(gpu, m, k) -> None:
    g = torch.Generator().manual_seed(m * 13 + k)
    x = (torch.randn(m, k, generator=g) * 3).to(BF).cuda()
    w = (torch.randn(k, generator=g) * 0.2 + 1).to(BF).cuda()
    if m > 2:
        x[1] = 0
    out, ws = gpu.rms_norm_q8k(x, w, 1e-5)
    assert out.dtype == BF
    xf = x.to(torch.float32)
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(BF) * w
    diff = (bf16_bits(out).to(torch.int32) - bf16_bits(ref).to(torch.int32)).abs()
    assert int(diff.max()) <= 1, "more than one bfloat16 ulp from torch's steps"
    assert float((diff == 0).float().mean()) > 0.98
    assert_q8k_of(gpu, ws, out)


@pytest.mark.parametrize("m,k", [(1, 14336), (16, 14336), (3, 1024)])
def test_silu_mul_bf16_equals_torch(gpu, m, k) -> None:
    g = torch.Generator().manual_seed(m + k)
    both = (torch.randn(m, 2 * k, generator=g) * 4).to(BF).cuda()
    both[0, :6] = torch.tensor([0.0, -0.0, 88.0, -88.0, 1e-30, -100.0])
    gate, up = both[:, :k], both[:, k:]  # the halves of a gate|up output, read in place
    out, ws = gpu.silu_mul_q8k(gate, up)
    want = TF.silu(gate) * up
    assert torch.equal(bf16_bits(out), bf16_bits(want))
    assert_q8k_of(gpu, ws, out)


class _Layer(nn.Module):
    """The projections and producers of a Llama-style layer in bfloat16 (q|k|v after a norm,
    gate|up after the same norm, down after SwiGLU)."""

    def __init__(self, k: int, ffn: int) -> None:
        super().__init__()
        self.w = {}

        def mk(t: int, n: int, kk: int, seed: int) -> DevicePackedLinear:
            w = S.packed_weight(t, n, kk, seed=seed)
            self.w[seed] = (t, w, n, kk)
            return DevicePackedLinear(dev(w), kk, t, dtype=BF)

        self.q_proj, self.k_proj = mk(D.Q4_K, 512, k, 1), mk(D.Q4_K, 128, k, 2)
        self.v_proj = mk(D.Q6_K, 128, k, 3)
        self.gate_proj, self.up_proj = mk(D.Q4_K, ffn, k, 4), mk(D.Q4_K, ffn, k, 5)
        self.down_proj = mk(D.Q6_K, k, ffn, 6)
        self.norm_w = torch.linspace(0.5, 1.5, k).to(BF).cuda()

    def forward(self, x: torch.Tensor, ops: HipFusedOps) -> list[torch.Tensor]:
        h = ops.rms_norm(x, self.norm_w, 1e-5)
        q, kk, v = project_shared(self, ("q_proj", "k_proj", "v_proj"), h)
        gate, up = project_shared(self, ("gate_proj", "up_proj"), h)
        hidden = ops.silu_mul(gate, up)
        return [h, q, kk, v, gate, up, hidden, self.down_proj(hidden)]


@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_bf16_layer_projections_bit_equal_oracle_with_handoff(gpu, oracle, monkeypatch,
                                                              tokens) -> None:
    """Every projection of the bfloat16 layer takes its producer's Q8_K blocks (the hand-off is
    hit) and equals, bit for bit, the oracle's matmul of the bfloat16 input it was given, rounded
    to bfloat16 by torch's cast."""
    k, ffn = 1024, 2048
    layer = _Layer(k, ffn)
    x = (torch.randn(1, tokens, k, generator=torch.Generator().manual_seed(tokens)) * 2).to(BF).cuda()
    hits = []
    claim = HANDOFF.claim

    def spy(t):
        ws = claim(t)
        hits.append(ws is not None)
        return ws

    monkeypatch.setattr(HANDOFF, "claim", spy)
    HipFusedOps.configure(True)
    try:
        h, q, kk, v, gate, up, hidden, down = layer(x, HipFusedOps.active())
    finally:
        HipFusedOps.configure(False)
    assert hits == [True, True, True], hits  # q|k|v, gate|up, down all on the producers' blocks
    for t_ in (h, q, kk, v, gate, up, hidden, down):
        assert t_.dtype == BF
    h2, hid2 = host(h.reshape(tokens, k).float()), host(hidden.reshape(tokens, ffn).float())
    for out, seed, inp in ((q, 1, h2), (kk, 2, h2), (v, 3, h2), (gate, 4, h2), (up, 5, h2),
                           (down, 6, hid2)):
        t, w, n, kk_ = layer.w[seed]
        want = torch.from_numpy(oracle.gemm(t, w, inp, n, kk_)).to(BF)
        assert torch.equal(bf16_bits(out.reshape(tokens, n)), want.view(torch.int16)), seed
    # the producers: silu * up is torch's bfloat16 steps bit for bit on the projections' outputs
    assert torch.equal(bf16_bits(hidden.reshape(tokens, ffn)),
                       bf16_bits(TF.silu(gate.reshape(tokens, ffn)) * up.reshape(tokens, ffn)))


def test_bf16_module_without_handoff_is_one_call(gpu) -> None:
    """A bfloat16 DevicePackedLinear on bfloat16 x: the result equals the float32 module's cast,
    and the module makes exactly one library call (no cast launches on either side)."""
    k, n = 4096, 1024
    w = dev(S.packed_weight(D.Q4_K, n, k, seed=11))
    mod = DevicePackedLinear(w, k, D.Q4_K, dtype=BF)
    mod32 = DevicePackedLinear(w, k, D.Q4_K, dtype=torch.float32)
    x = x_bf16(3, k, seed=12).reshape(1, 3, k)
    gpu.take_stats()
    y = mod(x)
    assert gpu.take_stats()[0] == 1
    assert y.dtype == BF and y.shape == (1, 3, n)
    assert torch.equal(bf16_bits(y), bf16_bits(mod32(x.to(torch.float32)).to(BF)))
    # a view that does not start on a 16-byte boundary is copied first
    xs = x_bf16(2, k + 8, seed=13)[:, 8:]
    assert torch.equal(bf16_bits(mod(xs)), bf16_bits(mod32(xs.float()).to(BF)))


# (type, N, K, M, taken by the kernel that reads bfloat16 x): its one- and three-row forms, a
# block count it has no form for, IQ4_XS (float activations), batched decode
NO_WS_CASES = [
    (D.Q4_K, 4096, 4096, 1, True), (D.Q6_K, 1024, 4096, 3, True), (D.Q8_0, 512, 2048, 2, True),
    (D.Q4_K, 700, 768, 1, False), (D.IQ4_XS, 1024, 4096, 1, False), (D.Q4_K, 4096, 4096, 16, False),
]


@pytest.mark.parametrize("t,n,k,m,taken", NO_WS_CASES)
def test_gemm_bf16_without_workspace(gpu, t, n, k, m, taken) -> None:
    """mxa_gemm_bf16 with a NULL workspace: a call the one-launch decode kernel takes gives the
    bits of the call with a workspace; any other returns MXA_ERR_WORKSPACE and launches nothing
    (y keeps its sentinel)."""
    from matricxon_amd.gemm import _stream

    assert gpu.fused_max_tokens == 3
    w = dev(S.packed_weight(t, n, k, seed=21 + m))
    xb = x_bf16(m, k, seed=22 + m)
    y = torch.full((m, n), 7.0, dtype=BF, device=w.device)
    status = gpu._lib.mxa_gemm_bf16(t, w.data_ptr(), xb.data_ptr(), y.data_ptr(), m, n, k, None, 0,
                                    _stream(w.device))
    torch.cuda.synchronize()
    if taken:
        assert status == 0
        assert torch.equal(bf16_bits(y), bf16_bits(gpu.matmul(t, w, xb.float(), n, k).to(BF)))
    else:
        assert status == -2
        assert bool((y == 7.0).all())


def test_raw_stream_handle_is_torchs_current_stream() -> None:
    """The launch stream the library is given is torch's current stream: the default one, one
    entered with `torch.cuda.stream`, for a device named with and without its index."""
    from matricxon_amd.gemm import _stream

    d = torch.device("cuda:0")
    assert _stream(d) == torch.cuda.current_stream(d).cuda_stream
    side = torch.cuda.Stream(d)
    with torch.cuda.stream(side):
        assert _stream(d) == side.cuda_stream
        assert _stream(torch.device("cuda")) == side.cuda_stream
    assert _stream(d) == torch.cuda.current_stream(d).cuda_stream != side.cuda_stream
