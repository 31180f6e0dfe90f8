"""Seeded synthetic packed weights and activations for the benchmark configurations.

Distributions follow the benchmark definition: f16 scale fields are float16(|N(0,1)| * sigma)
(about 0.5-1% of them land in the f16 subnormal range and are kept), quantized fields are
uniform over their full range, activations are float32 N(0,1). numpy `default_rng(seed)` (PCG64)
drives everything, so a (type, shape, seed) triple always gives the same bytes.
"""

import numpy as np

from matricxon_amd.quant_types import GEOMETRY, GGMLType


def _half_bytes(rng: np.random.Generator, n: int, sigma: float) -> np.ndarray:
    h = (np.abs(rng.standard_normal(n)) * sigma).astype(np.float16)
    return h.view(np.uint8).reshape(n, 2)


def _pack_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """(n, 8) six-bit scales and mins into the 12-byte Q4_K field, the inverse of ggml's
    get_scale_min_k4 (app/gguf/dequant/kquants.py:10-23)."""
    out = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    out[:, 0:4] = (sc[:, :4] & 0x3F) | ((sc[:, 4:] >> 4) << 6)
    out[:, 4:8] = (mn[:, :4] & 0x3F) | ((mn[:, 4:] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:] & 0x0F) | ((mn[:, 4:] & 0x0F) << 4)
    return out


def blocks_q8_0(rng: np.random.Generator, n_blocks: int, d_sigma: float = 0.02) -> np.ndarray:
    out = np.empty((n_blocks, 34), dtype=np.uint8)
    out[:, 0:2] = _half_bytes(rng, n_blocks, d_sigma)
    out[:, 2:] = rng.integers(-127, 128, size=(n_blocks, 32), dtype=np.int8).view(np.uint8)
    return out


def blocks_q4_k(rng: np.random.Generator, n_blocks: int, d_sigma: float = 0.01,
                dmin_sigma: float = 0.005) -> np.ndarray:
    out = np.empty((n_blocks, 144), dtype=np.uint8)
    out[:, 0:2] = _half_bytes(rng, n_blocks, d_sigma)
    out[:, 2:4] = _half_bytes(rng, n_blocks, dmin_sigma)
    sc = rng.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    out[:, 4:16] = _pack_k4(sc, mn)
    out[:, 16:] = rng.integers(0, 256, size=(n_blocks, 128), dtype=np.uint8)
    return out


def blocks_q6_k(rng: np.random.Generator, n_blocks: int, d_sigma: float = 0.005,
                sc_low: int = -64, sc_high: int = 63) -> np.ndarray:
    out = np.empty((n_blocks, 210), dtype=np.uint8)
    out[:, 0:192] = rng.integers(0, 256, size=(n_blocks, 192), dtype=np.uint8)
    out[:, 192:208] = rng.integers(sc_low, sc_high + 1, size=(n_blocks, 16),
                                   dtype=np.int8).view(np.uint8)
    out[:, 208:210] = _half_bytes(rng, n_blocks, d_sigma)
    return out


def blocks_iq4_xs(rng: np.random.Generator, n_blocks: int, d_sigma: float = 0.01) -> np.ndarray:
    """IQ4_XS blocks; the benchmark leaves sigma of d unspecified and fixes it at 0.01."""
    out = np.empty((n_blocks, 136), dtype=np.uint8)
    out[:, 0:2] = _half_bytes(rng, n_blocks, d_sigma)
    ls = rng.integers(0, 64, size=(n_blocks, 8), dtype=np.uint16)
    high = np.zeros(n_blocks, dtype=np.uint16)
    for ib in range(8):
        high |= (ls[:, ib] >> 4) << (2 * ib)
    out[:, 2:4] = high.view(np.uint8).reshape(n_blocks, 2)
    low = (ls & 0x0F).astype(np.uint8)
    out[:, 4:8] = low[:, 0::2] | (low[:, 1::2] << 4)
    out[:, 8:] = rng.integers(0, 256, size=(n_blocks, 128), dtype=np.uint8)
    return out


_MAKERS = {
    GGMLType.Q8_0: blocks_q8_0,
    GGMLType.Q4_K: blocks_q4_k,
    GGMLType.Q6_K: blocks_q6_k,
    GGMLType.IQ4_XS: blocks_iq4_xs,
}


def packed_weight(ggml_type: int, out_features: int, in_features: int, seed: int,
                  **kwargs) -> np.ndarray:
    """(out_features, row_bytes) uint8 packed rows of a random weight of `ggml_type`."""
    block, size = GEOMETRY[int(ggml_type)]
    n_blocks = out_features * (in_features // block)
    blocks = _MAKERS[GGMLType(int(ggml_type))](np.random.default_rng(seed), n_blocks, **kwargs)
    return blocks.reshape(out_features, (in_features // block) * size)


def activations(n_tokens: int, in_features: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((n_tokens, in_features), dtype=np.float32)


def integer_activations(n_tokens: int, in_features: int, seed: int) -> np.ndarray:
    """Integers in [-127, 127] with a +127 peak in every 256-value block: Q8_K quantizes them
    losslessly (d = 1, q = x), so a matmul on them is exact up to the fp32 folds
    (the reference's exact check, tests/unit/test_native_gemm.py:95-115)."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-127, 128, size=(n_tokens, in_features)).astype(np.float32)
    x[:, ::256] = 127.0
    return x


# The benchmark configurations (one seed each).
LLAMA3_8B_LAYER = (
    # (name, type, out_features, in_features)
    ("attn_q", GGMLType.Q4_K, 4096, 4096),
    ("attn_k", GGMLType.Q4_K, 1024, 4096),
    ("attn_v", GGMLType.Q6_K, 1024, 4096),
    ("attn_output", GGMLType.Q4_K, 4096, 4096),
    ("ffn_gate", GGMLType.Q4_K, 14336, 4096),
    ("ffn_up", GGMLType.Q4_K, 14336, 4096),
    ("ffn_down", GGMLType.Q6_K, 4096, 14336),
)
