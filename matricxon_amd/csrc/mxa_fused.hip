// Fused producers of the projections' activations: RMSNorm and SwiGLU's silu(gate) * up, each
// writing its result (float32, or bfloat16 for a bfloat16 layer) and the Q8_K blocks of that
// result in one pass, so that the projections that consume it (q|k|v and gate|up after a norm,
// down after SwiGLU) skip the quantize launch.
//
// Both take four values per thread, a wave per 256-value block, so that a call is one memory round
// trip and a short dependent chain (decode sizes are latency-bound): RMSNorm one workgroup of up
// to 1024 threads per row, silu * up one per 1024 values; the earlier 16-values-per-lane forms
// remain for operands that are not 16-byte aligned and for rows above 16384. The elementwise
// steps are the reference's, in its order
// (app/native/src/mx_fused_ops.c:6-17, 36-42): out = x * scale * w with scale = 1 / sqrtf(sum of
// squares / dim + eps), and out = g / (1 + expf(-g)) * u. The sum of squares is a tree over the
// workgroup (the reference's SIMD reduction has no fixed order either). Each 256-value block of the
// result is then quantized with the quantize kernel's own steps (q8k_part16, or q8k_part4 over a
// wave: the same amax, scale, rounding and sums), so the Q8_K blocks equal those of quantizing the
// fp32 result separately.
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

// Q8_K of one 256-value block held by a wave, four values per lane (lane l: values 4l .. 4l + 3):
// the steps of q8k_part16 (amax over the block from 0 with fmaxf, rintf of v * (127 / amax)
// clamped to +-127, int sums of 16, d = amax / 127) with the block maximum over the wave.
__device__ __forceinline__ void q8k_part4(const float (&v)[4], int lane, int8_t* qblk,
                                          int16_t* bsblk, float* dp) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = max16(amax);
  const auto lane_max = [&](int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, amax), l));
  };
  amax = fmaxf(fmaxf(lane_max(0), lane_max(16)), fmaxf(lane_max(32), lane_max(48)));
  int qv[4] = {0, 0, 0, 0};
  if (amax != 0.0f) {
    const float iscale = 127.0f / amax;
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = (int)fminf(fmaxf(rintf(v[i] * iscale), -127.0f), 127.0f);
  }
  *(uint32_t*)(qblk + 4 * lane) = (uint32_t)(qv[0] & 0xFF) | ((uint32_t)(qv[1] & 0xFF) << 8) |
                                   ((uint32_t)(qv[2] & 0xFF) << 16) | ((uint32_t)(qv[3] & 0xFF) << 24);
  const int bsum = quad_sum(qv[0] + qv[1] + qv[2] + qv[3]);  // values 16 (lane / 4) .. + 15
  if ((lane & 3) == 0) bsblk[lane >> 2] = (int16_t)bsum;
  if (lane == 0) *dp = amax / 127.0f;
}

constexpr int kRmsMaxThreads = 1024, kRmsMaxParts = 4;  // rows up to 16384 values

// RMSNorm of row blockIdx.x, four values per thread: thread t holds float4s t + T j (T threads,
// j < parts), all loaded before the sum of squares, so the row is read once.
__global__ __launch_bounds__(kRmsMaxThreads) void rms_norm_q8k_v4_kernel(
    const float* __restrict__ x, const float* __restrict__ w, float eps, float* __restrict__ out,
    int8_t* __restrict__ q, float* __restrict__ d, int16_t* __restrict__ bsums, int k) {
  __shared__ float part[kRmsMaxThreads / 64];
  const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, T = blockDim.x, n4 = k / 4;
  const int nb = k / QK;
  const float* xr = x + (size_t)r * k;
  float4 xv[kRmsMaxParts], wv[kRmsMaxParts];
#pragma unroll
  for (int j = 0; j < kRmsMaxParts; ++j) {
    const int i = t + T * j;
    if (i < n4) {
      xv[j] = *(const float4*)(xr + 4 * i);
      wv[j] = *(const float4*)(w + 4 * i);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kRmsMaxParts; ++j) {
    if (t + T * j < n4) {
      s = s + xv[j].x * xv[j].x;
      s = s + xv[j].y * xv[j].y;
      s = s + xv[j].z * xv[j].z;
      s = s + xv[j].w * xv[j].w;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s = s + __shfl_xor(s, o);
  if (lane == 0) part[t >> 6] = s;
  __syncthreads();
  float sum = 0.0f;
  for (int i = 0; i < T / 64; ++i) sum = sum + part[i];
  const float scale = 1.0f / sqrtf(sum / (float)k + eps);
#pragma unroll
  for (int j = 0; j < kRmsMaxParts; ++j) {
    const int i = t + T * j;
    if (i < n4) {  // uniform over the wave: n4 is a multiple of 64
      const float v[4] = {xv[j].x * scale * wv[j].x, xv[j].y * scale * wv[j].y,
                          xv[j].z * scale * wv[j].z, xv[j].w * scale * wv[j].w};
      if (out != nullptr) *(float4*)(out + (size_t)r * k + 4 * i) = float4{v[0], v[1], v[2], v[3]};
      const int b = i >> 6;
      q8k_part4(v, lane, q + (size_t)r * k + (size_t)b * QK, bsums + ((size_t)r * nb + b) * 16,
                d + (size_t)r * nb + b);
    }
  }
}

// silu(gate) * up of row blockIdx.x, float4 256 blockIdx.y + threadIdx.x of the row.
__global__ __launch_bounds__(256) void silu_mul_q8k_v4_kernel(
    const float* __restrict__ gate, const float* __restrict__ up, long long ld,
    float* __restrict__ out, int8_t* __restrict__ q, float* __restrict__ d,
    int16_t* __restrict__ bsums, int k) {
  const int r = blockIdx.x, i = 256 * (int)blockIdx.y + (int)threadIdx.x, lane = threadIdx.x & 63;
  if (i >= k / 4) return;  // uniform over the wave: k / 4 is a multiple of 64
  const float4 g4 = *(const float4*)(gate + (size_t)r * ld + 4 * i);
  const float4 u4 = *(const float4*)(up + (size_t)r * ld + 4 * i);
  const float g[4] = {g4.x, g4.y, g4.z, g4.w}, u[4] = {u4.x, u4.y, u4.z, u4.w};
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
  if (out != nullptr) *(float4*)(out + (size_t)r * k + 4 * i) = float4{v[0], v[1], v[2], v[3]};
  const int nb = k / QK, b = i >> 6;
  q8k_part4(v, lane, q + (size_t)r * k + (size_t)b * QK, bsums + ((size_t)r * nb + b) * 16,
            d + (size_t)r * nb + b);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Four bfloat16 values (8 bytes) as floats, exactly.
__device__ __forceinline__ void bf16x4_to_float(uint2 h, float (&v)[4]) {
  v[0] = bf16_to_float(h.x), v[1] = bf16_to_float(h.x >> 16);
  v[2] = bf16_to_float(h.y), v[3] = bf16_to_float(h.y >> 16);
}
__device__ __forceinline__ uint2 float4_to_bf16x4(const float (&v)[4]) {
  return uint2{(uint32_t)bf16_rne(v[0]) | (uint32_t)bf16_rne(v[1]) << 16,
               (uint32_t)bf16_rne(v[2]) | (uint32_t)bf16_rne(v[3]) << 16};
}

// RMSNorm of a bfloat16 layer, the steps of the reference's torch forward for a bfloat16 input
// and weight (app/architectures/layers.py:77-81): x widened to float32, variance = the mean of x^2
// (torch's mean multiplies the sum by 1 / dim), x * rsqrt(variance + eps) rounded to bfloat16,
// times the bfloat16 weight, rounded again. Row blockIdx.x, four values per thread (as
// rms_norm_q8k_v4_kernel); the Q8_K blocks are those of the bfloat16 result.
__global__ __launch_bounds__(kRmsMaxThreads) void rms_norm_q8k_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, float eps,
    uint16_t* __restrict__ out, int8_t* __restrict__ q, float* __restrict__ d,
    int16_t* __restrict__ bsums, int k) {
  __shared__ float part[kRmsMaxThreads / 64];
  const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, T = blockDim.x, n4 = k / 4;
  const int nb = k / QK;
  const uint16_t* xr = x + (size_t)r * k;
  float xv[kRmsMaxParts][4], wv[kRmsMaxParts][4];
#pragma unroll
  for (int j = 0; j < kRmsMaxParts; ++j) {
    const int i = t + T * j;
    if (i < n4) {
      bf16x4_to_float(*(const uint2*)(xr + 4 * i), xv[j]);
      bf16x4_to_float(*(const uint2*)(w + 4 * i), wv[j]);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kRmsMaxParts; ++j)
    if (t + T * j < n4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s = s + xv[j][e] * xv[j][e];
    }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s = s + __shfl_xor(s, o);
  if (lane == 0) part[t >> 6] = s;
  __syncthreads();
  float sum = 0.0f;
  for (int i = 0; i < T / 64; ++i) sum = sum + part[i];
  const float scale = rsqrtf(sum * (1.0f / (float)k) + eps);
#pragma unroll
  for (int j = 0; j < kRmsMaxParts; ++j) {
    const int i = t + T * j;
    if (i < n4) {  // uniform over the wave: n4 is a multiple of 64
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = bf16_to_float(bf16_rne(bf16_to_float(bf16_rne(xv[j][e] * scale)) * wv[j][e]));
      if (out != nullptr) *(uint2*)(out + (size_t)r * k + 4 * i) = float4_to_bf16x4(v);
      const int b = i >> 6;
      q8k_part4(v, lane, q + (size_t)r * k + (size_t)b * QK, bsums + ((size_t)r * nb + b) * 16,
                d + (size_t)r * nb + b);
    }
  }
}

// silu(gate) * up of a bfloat16 layer, the steps of torch's `F.silu(gate) * up` on bfloat16
// tensors (app/architectures/layers.py:53-57): g / (1 + exp(-g)) in float32 rounded to bfloat16,
// times up, rounded again. Row blockIdx.x, four values 256 blockIdx.y + threadIdx.x of the row;
// the Q8_K blocks are those of the bfloat16 result.
__global__ __launch_bounds__(256) void silu_mul_q8k_bf16_kernel(
    const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up, long long ld,
    uint16_t* __restrict__ out, int8_t* __restrict__ q, float* __restrict__ d,
    int16_t* __restrict__ bsums, int k) {
  const int r = blockIdx.x, i = 256 * (int)blockIdx.y + (int)threadIdx.x, lane = threadIdx.x & 63;
  if (i >= k / 4) return;  // uniform over the wave: k / 4 is a multiple of 64
  float g[4], u[4], v[4];
  bf16x4_to_float(*(const uint2*)(gate + (size_t)r * ld + 4 * i), g);
  bf16x4_to_float(*(const uint2*)(up + (size_t)r * ld + 4 * i), u);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    v[e] = bf16_to_float(bf16_rne(bf16_to_float(bf16_rne(g[e] / (1.0f + expf(-g[e])))) * u[e]));
  if (out != nullptr) *(uint2*)(out + (size_t)r * k + 4 * i) = float4_to_bf16x4(v);
  const int nb = k / QK, b = i >> 6;
  q8k_part4(v, lane, q + (size_t)r * k + (size_t)b * QK, bsums + ((size_t)r * nb + b) * 16,
            d + (size_t)r * nb + b);
}

}  // namespace

int launch_rms_norm_q8k_bf16(const uint16_t* x, const uint16_t* w, float eps, uint16_t* out,
                             const ActBuffers& a, int m_rows, int k, hipStream_t stream) {
  const int n4 = k / 4;
  if (n4 > kRmsMaxThreads * kRmsMaxParts || (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 7))
    return -1;
  hipLaunchKernelGGL(rms_norm_q8k_bf16_kernel, dim3(m_rows), dim3(min(n4, kRmsMaxThreads)), 0,
                     stream, x, w, eps, out, a.q, a.d, a.bsums, k);
  return 0;
}

int launch_silu_mul_q8k_bf16(const uint16_t* gate, const uint16_t* up, long long ld, uint16_t* out,
                             const ActBuffers& a, int m_rows, int k, hipStream_t stream) {
  if ((((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) & 7) || ld % 4 != 0) return -1;
  hipLaunchKernelGGL(silu_mul_q8k_bf16_kernel, dim3(m_rows, (k / 4 + 255) / 256), dim3(256), 0,
                     stream, gate, up, ld, out, a.q, a.d, a.bsums, k);
  return 0;
}

void launch_rms_norm_q8k(const float* x, const float* w, float eps, float* out, const ActBuffers& a,
                         int m_rows, int k, hipStream_t stream) {
  const int n4 = k / 4;
  const int threads = min(n4, kRmsMaxThreads);
  if (aligned16(x) && aligned16(w) && n4 <= kRmsMaxThreads * kRmsMaxParts) {
    hipLaunchKernelGGL(rms_norm_q8k_v4_kernel, dim3(m_rows), dim3(threads), 0, stream, x, w, eps,
                       out, a.q, a.d, a.bsums, k);
    return;
  }
  hipLaunchKernelGGL(rms_norm_q8k_kernel, dim3(m_rows), dim3(kFusedThreads), 0, stream, x, w, eps, out,
                     a.q, a.d, a.bsums, k);
}

void launch_silu_mul_q8k(const float* gate, const float* up, long long ld, float* out,
                         const ActBuffers& a, int m_rows, int k, hipStream_t stream) {
  if (aligned16(gate) && aligned16(up) && ld % 4 == 0) {
    hipLaunchKernelGGL(silu_mul_q8k_v4_kernel, dim3(m_rows, (k / 4 + 255) / 256), dim3(256), 0,
                       stream, gate, up, ld, out, a.q, a.d, a.bsums, k);
    return;
  }
  hipLaunchKernelGGL(silu_mul_q8k_kernel, dim3(m_rows, (k / QK + 15) / 16), dim3(kFusedThreads), 0,
                     stream, gate, up, ld, out, a.q, a.d, a.bsums, k);
}

}  // namespace mxa
