"""mxa_gemm_static, the no-allocation variant of mxa_gemm (its workspace is a per-device static
array), through the C ABI: each call equals mxa_gemm's result bit for bit, also when a second
call with a smaller input follows on the same scratch, and a call that needs more workspace than
the array holds is refused before any launch."""

import numpy as np
import pytest
import torch

from matricxon_amd import _lib
from matricxon_amd import synthetic as S
from matricxon_amd.gemm import _stream
from oracle import dequant as D
from tests.test_gpu_kernels import assert_within_tolerance, bits, dev, host

pytestmark = pytest.mark.gpu

SCRATCH = 16 << 20


def _static(lib, t, w, x, n, k):
    m = x.shape[0]
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    st = lib.mxa_gemm_static(t, w.data_ptr(), x.data_ptr(), y.data_ptr(), m, n, k,
                             _stream(y.device))
    assert st == 0, (st, lib.mxa_last_error())
    return y


# (type, N, K, first M, second smaller M): Q8_K workspace for K-quants above 3 rows, the bf16 split
# of x for IQ4_XS prefill, none for a one-row decode
CASES = [
    (D.Q4_K, 512, 4096, 16, 5),
    (D.Q6_K, 300, 2048, 64, 17),
    (D.Q8_0, 256, 1024, 9, 1),
    (D.IQ4_XS, 256, 4096, 48, 20),
    (D.Q4_K, 1000, 4096, 512, 40),
]


@pytest.mark.parametrize("t,n,k,m1,m2", CASES)
def test_static_equals_gemm_on_two_calls(gpu, oracle, t, n, k, m1, m2) -> None:
    lib = _lib.load()
    w_np = S.packed_weight(t, n, k, seed=80 + m1)
    w = dev(w_np)
    x1 = dev(S.activations(m1, k, seed=81))
    x2 = dev(S.activations(m2, k, seed=82))
    y1 = _static(lib, t, w, x1, n, k)
    y2 = _static(lib, t, w, x2, n, k)  # smaller input, same scratch, right after
    want1 = host(gpu.matmul(t, w, x1, n, k))
    want2 = host(gpu.matmul(t, w, x2, n, k))
    got1, got2 = host(y1), host(y2)
    assert np.array_equal(bits(got1), bits(want1))
    assert np.array_equal(bits(got2), bits(want2))
    assert_within_tolerance(got2, oracle.gemm(t, w_np, host(x2), n, k))


def test_static_refuses_a_workspace_beyond_the_array(gpu) -> None:
    lib = _lib.load()
    k, m = 4096, 1100  # IQ4_XS prefill: 4 * M * K bytes of split activations > 16 MiB
    assert lib.mxa_workspace_bytes(D.IQ4_XS, m, k) > SCRATCH
    w = dev(S.packed_weight(D.IQ4_XS, 64, k, seed=1))
    x = torch.zeros((m, k), dtype=torch.float32, device="cuda")
    y = torch.full((m, 64), 7.0, dtype=torch.float32, device="cuda")
    st = lib.mxa_gemm_static(D.IQ4_XS, w.data_ptr(), x.data_ptr(), y.data_ptr(), m, 64, k,
                             _stream(y.device))
    assert st == -2
    assert b"static scratch" in lib.mxa_last_error()
    assert bool((host(y) == 7.0).all())  # nothing was launched


@pytest.mark.parametrize("t,n,k,m", [(D.Q4_K, 1024, 4096, 1), (D.Q4_K, 512, 4096, 16),
                                     (D.IQ4_XS, 256, 4096, 20)])
def test_static_under_graph_capture(gpu, t, n, k, m) -> None:
    """A call captured into a HIP graph (after one eager call of the same shape on the device,
    which does the per-device set-up) replays to mxa_gemm's bits, replay after replay, with eager
    work of the program between the replays."""
    lib = _lib.load()
    w = dev(S.packed_weight(t, n, k, seed=90 + m))
    x = dev(S.activations(m, k, seed=91))
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    want = host(gpu.matmul(t, w, x, n, k))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        assert lib.mxa_gemm_static(t, w.data_ptr(), x.data_ptr(), y.data_ptr(), m, n, k,
                                   _stream(y.device)) == 0
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert np.array_equal(bits(host(y)), bits(want))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = lib.mxa_gemm_static(t, w.data_ptr(), x.data_ptr(), y.data_ptr(), m, n, k,
                                 _stream(y.device))
    assert st == 0, (st, lib.mxa_last_error())
    x2 = dev(S.activations(max(1, m // 2), k, seed=92))
    want2 = host(gpu.matmul(t, w, x2, n, k))
    for r in range(3):
        y.fill_(float("nan"))
        other = host(_static(lib, t, w, x2, n, k))  # eager call on the same scratch array
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(host(y)), bits(want)), f"replay {r}"
        assert np.array_equal(bits(other), bits(want2)), f"eager call before replay {r}"
    del graph
