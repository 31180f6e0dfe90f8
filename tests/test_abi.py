"""The C ABI without a GPU: the library loads next to torch's HIP runtime, exports every symbol
include/matricxon_amd.h declares, and its host-only queries and argument checks behave (no
kernel is launched by anything here)."""

import ctypes
import re

import pytest

from tests.conftest import REPO

HEADER = REPO / "include" / "matricxon_amd.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(mxa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from matricxon_amd import _lib

    return _lib.load()


def test_every_declared_symbol_is_exported(lib) -> None:
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    from matricxon_amd._lib import EXPORTS

    assert sorted(EXPORTS) == names


def test_only_torch_hip_runtime_is_mapped(lib) -> None:
    import torch

    maps = open("/proc/self/maps").read()
    hip = set(re.findall(r"/\S*libamdhip64\S*", maps))
    assert len(hip) == 1 and str(REPO) not in next(iter(hip))
    assert any(p.startswith(str(REPO / "matricxon_amd")) for p in
               re.findall(r"/\S*libmatricxon_amd\S*", maps))
    assert torch.__file__


def test_supports_and_sizes(lib) -> None:
    assert lib.mxa_supports(12, 3072) == 1
    assert lib.mxa_supports(12, 3000) == 0
    assert lib.mxa_supports(10, 3072) == 0  # Q2_K: not one of the four types
    assert lib.mxa_supports(8, 256) == 1 and lib.mxa_supports(8, 224) == 0
    assert lib.mxa_row_bytes(12, 4096) == 2304
    assert lib.mxa_row_bytes(14, 4096) == 3360
    assert lib.mxa_row_bytes(8, 4096) == 4352
    assert lib.mxa_row_bytes(23, 4096) == 2176
    assert lib.mxa_row_bytes(14, 14336) == 11760
    # Q8_K workspace: q (M*K) | d (M*nb*4) | bsums (M*nb*32), each 256-aligned
    assert lib.mxa_workspace_bytes(12, 16, 4096) == 65536 + 1024 + 8192
    assert lib.mxa_workspace_bytes(12, 5, 256) == 1280 + 256 + 256
    assert lib.mxa_workspace_bytes(12, 3, 4096) == 0  # quantized inside the matmul kernel
    assert lib.mxa_workspace_bytes(12, 4, 4096) == 16384 + 256 + 2048
    assert lib.mxa_workspace_bytes(23, 16, 4096) == 0  # IQ4_XS reads float activations
    assert lib.mxa_workspace_bytes(23, 17, 4096) == 17 * 4096 * 4  # prefill: bf16 hi/lo of x


def test_argument_errors_return_status_without_launching(lib) -> None:
    vp = ctypes.c_void_p
    a = vp(0x10000)  # a well-aligned stand-in address: nothing is dereferenced on these paths
    # unsupported type / shape -> -1
    assert lib.mxa_gemm(10, a, a, a, 1, 4, 4096, a, 1 << 20, None) == -1
    assert lib.mxa_gemm(12, a, a, a, 1, 4, 4000, a, 1 << 20, None) == -1
    assert lib.mxa_gemm(12, None, a, a, 1, 4, 4096, a, 1 << 20, None) == -1
    assert lib.mxa_gemm(12, a, a, a, 0, 4, 4096, a, 1 << 20, None) == -1
    # misaligned weights (dwords), activations or workspace (16-byte vectors) -> -1
    assert lib.mxa_gemm(12, vp(0x10002), a, a, 1, 4, 4096, a, 1 << 20, None) == -1
    assert lib.mxa_gemm(12, a, vp(0x10008), a, 1, 4, 4096, a, 1 << 20, None) == -1
    assert lib.mxa_gemm(12, a, a, a, 16, 4, 4096, vp(0x10004), 1 << 20, None) == -1
    assert lib.mxa_quantize_q8_k(vp(0x10004), 2, 512, a, 1 << 20, None) == -1
    # workspace too small -> -2
    assert lib.mxa_gemm(12, a, a, a, 16, 4, 4096, a, 1000, None) == -2
    assert lib.mxa_gemm(12, a, a, a, 16, 4, 4096, None, 1 << 20, None) == -2
    assert lib.mxa_gemm(12, a, a, a, 5, 4, 4096, a, 1000, None) == -2
    assert lib.mxa_quantize_q8_k(a, 2, 512, a, 10, None) == -2
    assert lib.mxa_dequantize(11, a, 4, a, None) == -1
    assert lib.mxa_dequant_rows(12, a, 10, a, 2, 300, a, None) == -1
    # fp32-activation GEMV: unsupported type / shape, null or misaligned operands -> -1
    assert lib.mxa_gemv_f32(10, a, a, a, 1, 4, 4096, None) == -1
    assert lib.mxa_gemv_f32(12, a, a, a, 1, 4, 4000, None) == -1
    assert lib.mxa_gemv_f32(14, a, None, a, 1, 4, 4096, None) == -1
    assert lib.mxa_gemv_f32(8, a, a, a, 0, 4, 4096, None) == -1
    assert lib.mxa_gemv_f32(23, a, vp(0x10008), a, 1, 4, 4096, None) == -1
    assert lib.mxa_gemv_f32(12, vp(0x10002), a, a, 1, 4, 4096, None) == -1
    n = 5
    types = (ctypes.c_int * n)(*([12] * n))
    assert lib.mxa_gemm_multi(n, types, a, a, a, a, 1, 4096, a, 1 << 20, None) == -1
    assert lib.mxa_last_error() == b""


def test_build_info(lib) -> None:
    assert b"gfx950" in lib.mxa_build_info()


def test_modules_fail_loudly_off_gpu() -> None:
    """No CPU fallback: host tensors are rejected before anything is launched."""
    import torch

    from matricxon_amd.gemm import HipGemm

    g = HipGemm.get()
    w = torch.zeros((4, 288), dtype=torch.uint8)
    with pytest.raises(ValueError, match="HIP device"):
        g.matmul(12, w, torch.zeros(1, 512), 4, 512)


def test_dequant_rows_support_query(lib) -> None:
    for t in (8, 12, 14, 23):
        assert lib.mxa_supports_dequant_rows(t, 4096) == 1
    assert lib.mxa_supports_dequant_rows(12, 4000) == 0
    assert lib.mxa_supports_dequant_rows(10, 4096) == 0


def test_fused_max_tokens_moves_the_workspace_crossover(lib) -> None:
    """`mx_set_fused_max_tokens` (app/native/src/mx_gemm.c:11-16): rows up to the crossover take
    the decode kernel (no Q8_K workspace), more rows quantize into the workspace."""
    assert lib.mxa_fused_max_tokens() == 3
    try:
        lib.mxa_set_fused_max_tokens(1)
        assert lib.mxa_fused_max_tokens() == 1
        assert lib.mxa_workspace_bytes(12, 1, 4096) == 0
        assert lib.mxa_workspace_bytes(12, 2, 4096) == 8192 + 256 + 1024
        lib.mxa_set_fused_max_tokens(0)
        assert lib.mxa_workspace_bytes(12, 1, 4096) == 4096 + 256 + 512
        lib.mxa_set_fused_max_tokens(99)  # clamped to the decode kernel's 4 rows
        assert lib.mxa_fused_max_tokens() == 4
        assert lib.mxa_workspace_bytes(12, 4, 4096) == 0
        assert lib.mxa_workspace_bytes(23, 17, 4096) == 17 * 4096 * 4  # IQ4_XS unaffected
        lib.mxa_set_fused_max_tokens(-5)
        assert lib.mxa_fused_max_tokens() == 0
    finally:
        lib.mxa_set_fused_max_tokens(3)


def test_fp32_gemv_registry_and_backend_setting(monkeypatch) -> None:
    """The Numba-registry mirror (quantized_gemv_registry.py:63-93) and MATRICXON_GEMV_BACKEND."""
    import torch

    from matricxon_amd import device_packed as DP
    from matricxon_amd.quantized_gemv import GEMV_KERNELS, has_gemv_kernel, qgemv_q6_k

    assert {t: size for t, (_, size) in GEMV_KERNELS.items()} == {8: 34, 12: 144, 14: 210, 23: 136}
    assert has_gemv_kernel(12) and not has_gemv_kernel(2) and not has_gemv_kernel(10)
    with pytest.raises(ValueError, match="multiple of block_size"):
        qgemv_q6_k(torch.zeros(300), torch.zeros(210, dtype=torch.uint8), 1, 300)
    monkeypatch.delenv("MATRICXON_GEMV_BACKEND", raising=False)
    assert DP.gemv_backend() == "native"
    monkeypatch.setenv("MATRICXON_GEMV_BACKEND", "Numba")
    assert DP.gemv_backend() == "numba"
    monkeypatch.setenv("MATRICXON_GEMV_BACKEND", "triton")
    with pytest.raises(ValueError, match="MATRICXON_GEMV_BACKEND"):
        DP.gemv_backend()
    g = DP.HipGemm.get()
    with pytest.raises(ValueError, match="HIP device"):
        g.gemv_f32(14, torch.zeros((1, 210), dtype=torch.uint8), torch.zeros(1, 256), 1, 256)


def test_build_refuses_scratch_in_register_load_kernels() -> None:
    """mxa_bwave.hip's kernels load into registers from inline assembly and wait themselves, so
    the build must refuse any of them that spills: the parser of hipcc's resource remarks names
    exactly the kernels with a nonzero scratch size."""
    from matricxon_amd import build

    assert "mxa_bwave.hip" in build.NO_SCRATCH
    remarks = "\n".join([
        "x.hip:9:1: remark: Function Name: _Zkeep [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark: Function Name: _Zspill [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     VGPRs: 128 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:9:1: remark:     ScratchSize [bytes/lane]: 228 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build.scratch_users(remarks) == ["_Zspill (228 bytes/lane)"]
    assert build.scratch_users("") == []
