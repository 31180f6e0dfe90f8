// Fused producers of the projections' activations: RMSNorm and SwiGLU's silu(gate) * up, each
// writing its fp32 result and the Q8_K blocks of that result in one pass, so that the projections
// that consume it (q|k|v and gate|up after a norm, down after SwiGLU) skip the quantize launch.
//
// RMSNorm: one workgroup (256 threads) per row; silu * up: one per 16 blocks of a row. The elementwise steps are the reference's, in its order
// (app/native/src/mx_fused_ops.c:6-17, 36-42): out = x * scale * w with scale = 1 / sqrtf(sum of
// squares / dim + eps), and out = g / (1 + expf(-g)) * u. The sum of squares is a tree over the
// workgroup (the reference's SIMD reduction has no fixed order either). Each 256-value block of the
// result is then quantized by 16 lanes with q8k_part16, the quantize kernel's own steps, so the
// Q8_K blocks equal those of quantizing the fp32 result separately.
#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

constexpr int kFusedThreads = 256;

// Blocks b0, b0 + 16, ... below nb of a row: the 16 values of lane part p of block b are produced
// by f(i) for element i, written to out (if any) and quantized into the row's Q8_K blocks.
template <class Fn>
__device__ __forceinline__ void emit_blocks(int b0, int nb, float* __restrict__ out_row, int8_t* qrow,
                                            int16_t* bsrow, float* drow, Fn f) {
  const int p = threadIdx.x & 15;
  // 16 blocks per pass, one per 16-lane DPP row; the rows of a pass stay whole (b is uniform
  // over them), as q8k_part16 needs
  for (int b = b0 + ((int)threadIdx.x >> 4); b < nb; b += kFusedThreads / 16) {
    const int base = b * QK + 16 * p;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = f(base + i);
    if (out_row != nullptr) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *(float4*)(out_row + base + 4 * i) = float4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    }
    q8k_part16(v, p, qrow + (size_t)b * QK, bsrow + (size_t)b * 16, drow + b);
  }
}

__global__ __launch_bounds__(kFusedThreads) void rms_norm_q8k_kernel(
    const float* __restrict__ x, const float* __restrict__ w, float eps, float* __restrict__ out,
    int8_t* __restrict__ q, float* __restrict__ d, int16_t* __restrict__ bsums, int k) {
  __shared__ float part[kFusedThreads / 64];
  const int r = blockIdx.x, nb = k / QK;
  const float* xr = x + (size_t)r * k;
  // sum of x^2: float4 i of the row by thread i mod 256, then the wave (xor butterflies) and the
  // workgroup (LDS)
  float s = 0.0f;
  for (int i = threadIdx.x; i < k / 4; i += kFusedThreads) {
    const float4 v = *(const float4*)(xr + 4 * i);
    s = s + v.x * v.x;
    s = s + v.y * v.y;
    s = s + v.z * v.z;
    s = s + v.w * v.w;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s = s + __shfl_xor(s, o);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const float sum = (part[0] + part[1]) + (part[2] + part[3]);
  const float scale = 1.0f / sqrtf(sum / (float)k + eps);
  emit_blocks(0, nb, out != nullptr ? out + (size_t)r * k : nullptr, q + (size_t)r * k,
              bsums + (size_t)r * nb * 16, d + (size_t)r * nb,
              [&](int i) { return xr[i] * scale * w[i]; });
}

// Row blockIdx.x, blocks 16 * blockIdx.y .. + 15 (one pass of the workgroup); gate and up rows are
// ld floats apart (they may be the two halves of one gate|up output).
__global__ __launch_bounds__(kFusedThreads) void silu_mul_q8k_kernel(
    const float* __restrict__ gate, const float* __restrict__ up, long long ld,
    float* __restrict__ out, int8_t* __restrict__ q, float* __restrict__ d,
    int16_t* __restrict__ bsums, int k) {
  const int r = blockIdx.x, nb = k / QK;
  const float* gr = gate + (size_t)r * ld;
  const float* ur = up + (size_t)r * ld;
  const int b0 = 16 * (int)blockIdx.y;
  emit_blocks(b0, min(nb, b0 + 16), out != nullptr ? out + (size_t)r * k : nullptr,
              q + (size_t)r * k, bsums + (size_t)r * nb * 16, d + (size_t)r * nb, [&](int i) {
                const float g = gr[i];
                return g / (1.0f + expf(-g)) * ur[i];
              });
}

}  // namespace

void launch_rms_norm_q8k(const float* x, const float* w, float eps, float* out, const ActBuffers& a,
                         int m_rows, int k, hipStream_t stream) {
  hipLaunchKernelGGL(rms_norm_q8k_kernel, dim3(m_rows), dim3(kFusedThreads), 0, stream, x, w, eps, out,
                     a.q, a.d, a.bsums, k);
}

void launch_silu_mul_q8k(const float* gate, const float* up, long long ld, float* out,
                         const ActBuffers& a, int m_rows, int k, hipStream_t stream) {
  hipLaunchKernelGGL(silu_mul_q8k_kernel, dim3(m_rows, (k / QK + 15) / 16), dim3(kFusedThreads), 0,
                     stream, gate, up, ld, out, a.q, a.d, a.bsums, k);
}

}  // namespace mxa
