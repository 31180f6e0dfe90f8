"""numpy float32 restatement of the reference dequantizers and of the Q8_K activation quantizer.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every function takes `blocks`, a `(n_blocks, type_size)` uint8 array (GGUF block order), and
returns the flat float32 values. Each arithmetic step is its own numpy ufunc call on float32
arrays, so every intermediate is rounded to float32 exactly where the reference rounds it (no
fused multiply-add): that makes the results bit-exact with the reference `QuantStrategy`
classes, which the packed GPU path (`TorchDequantizer`) mirrors bit for bit.
"""

import numpy as np

Q8_0, Q4_K, Q6_K, IQ4_XS = 8, 12, 14, 23

# (elements per block, bytes per block), app/gguf/dequant/legacy.py:13-20, kquants.py:26-32,115-121,
# iq_ternary.py:51-60.
GEOMETRY = {Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), IQ4_XS: (256, 136)}

# The fixed non-linear IQ4 grid (app/gguf/dequant/iq_ternary.py:18-21): ggml's kvalues_iq4nl.
IQ4_GRID = np.array(
    [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.float32
)


def _f16_at(blocks: np.ndarray, offset: int) -> np.ndarray:
    """Little-endian IEEE half at byte `offset` of each block, widened exactly to float32
    (subnormal halves become normal floats), shape (n_blocks, 1)."""
    raw = np.ascontiguousarray(blocks[:, offset : offset + 2]).view("<f2")
    return raw.astype(np.float32).reshape(-1, 1)


def k4_scales_mins(scales12: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The 8 six-bit (scale, min) pairs of a Q4_K block from its 12 packed bytes
    (app/gguf/dequant/kquants.py:10-23): pairs 0-3 are the low 6 bits of bytes j and j+4; pairs
    4-7 take byte j+4's low / high nibble plus the top two bits of bytes j-4 / j."""
    s = scales12.astype(np.uint8)
    sc = np.empty((s.shape[0], 8), dtype=np.uint8)
    mn = np.empty((s.shape[0], 8), dtype=np.uint8)
    sc[:, :4] = s[:, 0:4] & 0x3F
    mn[:, :4] = s[:, 4:8] & 0x3F
    sc[:, 4:] = (s[:, 8:12] & 0x0F) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def pack_k4_scales_mins(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of `k4_scales_mins`: (n, 8) six-bit scales and mins -> (n, 12) packed bytes."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    out[:, 0:4] = (sc[:, :4] & 0x3F) | ((sc[:, 4:] >> 4) << 6)
    out[:, 4:8] = (mn[:, :4] & 0x3F) | ((mn[:, 4:] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:] & 0x0F) | ((mn[:, 4:] & 0x0F) << 4)
    return out


def dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    """value = qs * d (app/gguf/dequant/legacy.py:22-29)."""
    d = _f16_at(blocks, 0)
    qs = np.ascontiguousarray(blocks[:, 2:34]).view(np.int8).astype(np.float32)
    return (qs * d).reshape(-1)


def dequant_q4_k(blocks: np.ndarray) -> np.ndarray:
    """value = (d * sc) * q - (dmin * m), in that rounding order (kquants.py:34-64). Element
    order: for chunk c = 0..3, the 32 low nibbles of qs[32c:32c+32] (sub-block 2c), then the 32
    high nibbles (sub-block 2c+1)."""
    n = blocks.shape[0]
    d = _f16_at(blocks, 0).reshape(n, 1, 1, 1)
    dmin = _f16_at(blocks, 2).reshape(n, 1, 1, 1)
    sc, mn = k4_scales_mins(blocks[:, 4:16])
    sc = sc.astype(np.float32).reshape(n, 4, 2, 1)
    mn = mn.astype(np.float32).reshape(n, 4, 2, 1)
    qs = blocks[:, 16:144].reshape(n, 4, 1, 32)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.float32)  # (n, chunk, half, 32)
    scaled = d * sc
    mins = dmin * mn
    return (scaled * q - mins).reshape(-1)


def q6_k_codes(blocks: np.ndarray) -> np.ndarray:
    """The 256 unsigned 6-bit codes u = q + 32 of each Q6_K block, in element order, int32
    (kquants.py:138-159): for half h, lane l < 32 with L = ql[64h:], H = qh[32h:], elements
    128h + l, +32, +64, +96 take (L[l] & 15 | (H[l] & 3) << 4), (L[l+32] & 15 | (H[l] >> 2 & 3) << 4),
    (L[l] >> 4 | (H[l] >> 4 & 3) << 4), (L[l+32] >> 4 | (H[l] >> 6) << 4)."""
    n = blocks.shape[0]
    ql = blocks[:, 0:128].reshape(n, 2, 2, 32).astype(np.int32)  # (n, half, lo/hi 32, lane)
    qh = blocks[:, 128:192].reshape(n, 2, 1, 32).astype(np.int32)
    low, high = ql & 0x0F, ql >> 4
    groups = np.stack(
        [
            low[:, :, 0] | ((qh[:, :, 0] & 3) << 4),
            low[:, :, 1] | (((qh[:, :, 0] >> 2) & 3) << 4),
            high[:, :, 0] | (((qh[:, :, 0] >> 4) & 3) << 4),
            high[:, :, 1] | (((qh[:, :, 0] >> 6) & 3) << 4),
        ],
        axis=2,
    )  # (n, half, group, lane)
    return groups.reshape(n, 256)


def dequant_q6_k(blocks: np.ndarray) -> np.ndarray:
    """value = (d * sc) * (u - 32) with a signed int8 scale per 16 elements (kquants.py:123-162)."""
    n = blocks.shape[0]
    d = _f16_at(blocks, 208)
    sc = np.ascontiguousarray(blocks[:, 192:208]).view(np.int8).astype(np.float32)
    scale = np.repeat(sc, 16, axis=1)  # (n, 256): element e uses sc[e // 16]
    q = q6_k_codes(blocks).astype(np.float32) - np.float32(32.0)
    return ((d * scale) * q).reshape(-1)


def iq4_xs_sub_scales(blocks: np.ndarray) -> np.ndarray:
    """The 8 six-bit sub-block scales ls (before the -32 offset) of each IQ4_XS block, int32
    (iq_ternary.py:78-81): low nibble from scales_l[ib/2] (nibble ib%2), top 2 bits from
    scales_h bits 2ib..2ib+1."""
    n = blocks.shape[0]
    scales_h = blocks[:, 2].astype(np.int32) | (blocks[:, 3].astype(np.int32) << 8)
    scales_l = blocks[:, 4:8].astype(np.int32)
    ib = np.arange(8)
    low = (scales_l[:, ib // 2] >> (4 * (ib % 2))) & 0x0F
    high = ((scales_h.reshape(n, 1) >> (2 * ib)) & 3) << 4
    return low | high


def dequant_iq4_xs(blocks: np.ndarray) -> np.ndarray:
    """value = (d * (ls - 32)) * grid[idx]; sub-block ib's 32 elements are the low nibbles of
    qs[16ib:16ib+16] then their high nibbles (iq_ternary.py:62-90)."""
    n = blocks.shape[0]
    d = _f16_at(blocks, 0)
    ls = iq4_xs_sub_scales(blocks)
    dl = (d * (ls - 32).astype(np.float32)).reshape(n, 8, 1)
    qs = blocks[:, 8:136].reshape(n, 8, 16)
    grid = np.concatenate([IQ4_GRID[qs & 0x0F], IQ4_GRID[qs >> 4]], axis=2)  # (n, 8, 32)
    return (dl * grid).reshape(-1)


_DEQUANT = {Q8_0: dequant_q8_0, Q4_K: dequant_q4_k, Q6_K: dequant_q6_k, IQ4_XS: dequant_iq4_xs}


def dequantize(ggml_type: int, blocks: np.ndarray) -> np.ndarray:
    """Flat float32 values of `blocks` ((n_blocks, type_size) uint8, or flat bytes)."""
    _, type_size = GEOMETRY[ggml_type]
    blocks = np.asarray(blocks, dtype=np.uint8).reshape(-1, type_size)
    return _DEQUANT[ggml_type](blocks)


def dequantize_matrix(ggml_type: int, packed: np.ndarray, out_features: int, in_features: int):
    """(out_features, in_features) float32 weight from `packed` rows."""
    return dequantize(ggml_type, packed).reshape(out_features, in_features)


def quantize_q8_k(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Q8_K activation quantization of (M, K) float32 `x` (app/native/src/mx_common.c:42-69),
    per 256-value block: amax = max |x| (an all-zero block quantizes to zeros with d = 0);
    iscale = 127 / amax and d = amax / 127, both correctly-rounded float32 divisions;
    q = clamp(round_half_even(x * iscale), -127, 127); bsums = sums of q over 16 values.
    Returns (q int8 (M, K), d float32 (M, K/256), bsums int16 (M, K/256, 16))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    xb = x.reshape(m, k // 256, 256)
    ax = np.abs(xb)
    # `ax > amax ? ax : amax` from 0 never picks a NaN
    amax = np.max(np.where(np.isnan(ax), np.float32(0.0), ax), axis=2)  # (m, nb)
    safe = np.where(amax == 0, np.float32(1.0), amax).astype(np.float32)
    iscale = (np.float32(127.0) / safe).astype(np.float32)
    with np.errstate(invalid="ignore"):
        scaled = (xb * iscale[:, :, None]).astype(np.float32)
    # lrintf of a NaN (inf * 0 included) is INT_MIN on x86, which the clamp turns into -127
    rounded = np.where(np.isnan(scaled), np.float32(-128.0), np.rint(scaled))
    q = np.clip(rounded, -127, 127).astype(np.int32)
    q[amax == 0] = 0
    d = (amax / np.float32(127.0)).astype(np.float32)
    bsums = q.reshape(m, k // 256, 16, 16).sum(axis=3).astype(np.int16)
    return q.reshape(m, k).astype(np.int8), d, bsums


def dequantize_q8_k(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """float64 values q * d of Q8_K activations (M, K) - what the integer dot products see."""
    m, k = q.shape
    return (q.reshape(m, k // 256, 256).astype(np.float64) * d[:, :, None]).reshape(m, k)
