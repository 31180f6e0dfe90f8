"""Device counterparts of the reference's fp32-activation GEMVs (the `gemv_backend = "numba"`
kernels): y = x @ W.T with x kept in float32, for a packed weight W that stays packed in device
memory.

* `qgemv_q4_k`, `qgemv_q6_k` (app/gguf/dequant/quantized_gemv.py:90-112, :164-180),
  `qgemv_q8_0` (app/gguf/dequant/quantized_gemv_legacy.py:183-194) and `qgemv_iq4_xs`
  (app/gguf/dequant/quantized_gemv_iq_ternary.py:91-107): same argument meaning,
  `(x (in_features,), raw, out_features, in_features) -> (out_features,) float32`, and the same
  `ValueError` when in_features is not a multiple of 256. `raw` is the packed bytes on the device
  (a uint8 tensor, flat or (out_features, row_bytes)) instead of a host memoryview; x and y live on
  that device.
* `GEMV_KERNELS` / `has_gemv_kernel` (app/gguf/dequant/quantized_gemv_registry.py:63-93):
  `{ggml_type: (gemv_fn, type_size)}` for the four types computed here.

Unlike the default path (`HipGemm.matmul`), x is never quantized to Q8_K: each weight value is its
dequantized float (d * sc * q - dmin * m) multiplied with the unquantized activation, the
numerics of the Numba kernels. The order of float additions is the kernel's own (the reference
compiles with fastmath and 2-4 accumulators, which fixes no order either); results agree with the
float64 product of the dequantized weight and x to float32 accuracy.
"""

import torch

from matricxon_amd.gemm import HipGemm
from matricxon_amd.quant_types import GEOMETRY

_QK_K = 256
_Q8_0, _Q4_K, _Q6_K, _IQ4_XS = 8, 12, 14, 23


def _require_divisible(in_features: int) -> int:
    """quantized_gemv.py:34-37: the block count of a row, or ValueError."""
    if in_features % _QK_K != 0:
        raise ValueError(f"in_features={in_features} is not a multiple of block_size={_QK_K}")
    return in_features // _QK_K


def _qgemv_of(ggml_type: int, name: str, weight: str):
    """The reference-named GEMV for one type: (x, raw, out_features, in_features) -> y."""

    def qgemv(x: torch.Tensor, raw: torch.Tensor, out_features: int,
              in_features: int) -> torch.Tensor:
        _require_divisible(in_features)
        gemm = HipGemm.get()
        packed = raw.reshape(out_features, gemm.row_bytes(ggml_type, in_features))
        y = gemm.gemv_f32(ggml_type, packed, x.reshape(1, in_features), out_features, in_features)
        return y.reshape(out_features)

    qgemv.__name__ = qgemv.__qualname__ = name
    qgemv.__doc__ = f"{weight} weight: y = x @ W.T, x in float32."
    return qgemv


qgemv_q4_k = _qgemv_of(_Q4_K, "qgemv_q4_k", "Q4_K (144-byte blocks of 256 values)")
qgemv_q6_k = _qgemv_of(_Q6_K, "qgemv_q6_k", "Q6_K (210-byte blocks of 256 values)")
qgemv_q8_0 = _qgemv_of(_Q8_0, "qgemv_q8_0", "Q8_0 (34-byte blocks of 32 values)")
qgemv_iq4_xs = _qgemv_of(_IQ4_XS, "qgemv_iq4_xs", "IQ4_XS (136-byte blocks of 256 values)")


GEMV_KERNELS: dict[int, tuple[callable, int]] = {
    _Q8_0: (qgemv_q8_0, GEOMETRY[_Q8_0][1]),
    _Q4_K: (qgemv_q4_k, GEOMETRY[_Q4_K][1]),
    _Q6_K: (qgemv_q6_k, GEOMETRY[_Q6_K][1]),
    _IQ4_XS: (qgemv_iq4_xs, GEOMETRY[_IQ4_XS][1]),
}


def has_gemv_kernel(ggml_type: int) -> bool:
    return int(ggml_type) in GEMV_KERNELS
