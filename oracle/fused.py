"""numpy float32 restatement of the reference's fused producer ops (RMSNorm, SwiGLU's silu * up).
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The elementwise steps round to float32 where the reference's C rounds them. The reference sums the
squares of a row with an OpenMP SIMD reduction, whose order is the compiler's; here the sum is
taken in float64 and rounded once, so results agree with the reference C (and with the device's
tree sum) to a few float32 ulps, not bit for bit.
"""

import numpy as np


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """out[r] = x[r] * (1 / sqrtf(sum(x[r]^2) / dim + eps)) * w, as `mx_rms_norm`
    (app/native/src/mx_fused_ops.c:6-17): the product (x * scale) * w in that order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    dim = x.shape[-1]
    ss = np.float32(np.sum(x.astype(np.float64) ** 2, axis=-1))
    mean = np.float32(ss / np.float32(dim))
    scale = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(eps)), dtype=np.float32)
    return (x * scale[..., None]).astype(np.float32) * w


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """out = g / (1 + expf(-g)) * u elementwise, as `mx_silu_mul` (mx_fused_ops.c:36-42)."""
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-g, dtype=np.float32)
    return (g / (np.float32(1.0) + e)).astype(np.float32) * u
