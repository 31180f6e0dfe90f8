"""matricxon_amd: the quantized-native matmul of Matricxon (fused dequantize-and-multiply over
packed GGUF blocks: Q8_0, Q4_K, Q6_K, IQ4_XS) as hand-written HIP kernels for AMD Instinct MI355X
(gfx950), behind the reference's `MATRICXON_GPU_WEIGHT_MODE=packed` module interface.

Importing the package loads nothing native; `HipGemm.get()` (or constructing a module) loads
libmatricxon_amd.so and fails loudly when it is not built.
"""

from matricxon_amd.quant_types import GEOMETRY, GGMLType, row_bytes

__all__ = ["GEOMETRY", "GGMLType", "row_bytes"]
