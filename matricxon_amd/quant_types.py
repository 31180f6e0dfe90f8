"""GGML type ids and block geometry of the four packed types this library computes on the GPU.

Type ids are ggml's (app/gguf/constants.py:24-59 `GGMLQuantizationType`); geometry is
(elements per block, bytes per block) as the reference strategies declare it
(app/gguf/dequant/legacy.py:13-20, kquants.py:26-32,115-121, iq_ternary.py:51-60).
"""

from enum import IntEnum


class GGMLType(IntEnum):
    Q8_0 = 8
    Q4_K = 12
    Q6_K = 14
    IQ4_XS = 23


GEOMETRY: dict[int, tuple[int, int]] = {
    GGMLType.Q8_0: (32, 34),
    GGMLType.Q4_K: (256, 144),
    GGMLType.Q6_K: (256, 210),
    GGMLType.IQ4_XS: (256, 136),
}

# Every type here needs in_features % 256 == 0, Q8_0 included: its activations are quantized in
# 256-value Q8_K blocks (app/native/src/mx_gemm.c:114-121).
SUPER_BLOCK = 256


def row_bytes(ggml_type: int, in_features: int) -> int:
    block, size = GEOMETRY[int(ggml_type)]
    return (in_features // block) * size


def geometry(ggml_type: int) -> tuple[int, int]:
    """`(block_size, type_size)`, as `TorchDequantizer.geometry` (torch_dequant.py:228-232)."""
    return GEOMETRY[int(ggml_type)]
