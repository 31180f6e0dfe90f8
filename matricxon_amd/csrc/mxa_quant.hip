// Q8_K activation quantization and bit-exact dequantization of packed GGUF blocks.
//
// Compiled with -ffp-contract=off: every float multiply and subtract below rounds on its own,
// in the order the reference's numpy dequantizers use, so results are bit-identical to them.
#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {

// 16 lanes per (row m, 256-value block b), four blocks per wave; lane part p owns elements
// 16p..16p+15 (q8k_part16 in mxa_kernels.hpp does the arithmetic).
// x is float32, or bfloat16 (BF16; widened exactly before the same steps).
template <bool BF16>
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const void* __restrict__ x,
                                                           int8_t* __restrict__ q,
                                                           float* __restrict__ d,
                                                           int16_t* __restrict__ bsums, int m_rows,
                                                           int k, int nb) {
  const int blk = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int p = threadIdx.x & 15;
  if (blk >= m_rows * nb) return;  // whole 16-lane rows leave together (the DPP max stays in a row)
  const int m = blk / nb, b = blk - m * nb;
  const size_t base = (size_t)m * k + (size_t)b * QK + 16 * p;
  float v[16];
  if constexpr (BF16) {
    const uint16_t* xh = (const uint16_t*)x + base;
    const uint4 a = *(const uint4*)xh, c = *(const uint4*)(xh + 8);
    const uint32_t hv[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = bf16_to_float(hv[i]);
      v[2 * i + 1] = bf16_to_float(hv[i] >> 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 f = *((const float4*)x + base / 4 + i);
      v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
    }
  }
  q8k_part16(v, p, q + (size_t)m * k + (size_t)b * QK, bsums + ((size_t)m * nb + b) * 16,
             d + (size_t)m * nb + b);
}

void launch_quantize_q8k(const float* x, const ActBuffers& a, int m_rows, int k,
                         hipStream_t stream) {
  const int nb = k / QK;
  const int blocks = m_rows * nb;
  const int grid = (blocks + 15) / 16;
  hipLaunchKernelGGL(quantize_q8k_kernel<false>, dim3(grid), dim3(256), 0, stream, x, a.q, a.d,
                     a.bsums, m_rows, k, nb);
}

void launch_quantize_q8k_bf16(const uint16_t* x, const ActBuffers& a, int m_rows, int k,
                              hipStream_t stream) {
  const int nb = k / QK;
  const int blocks = m_rows * nb;
  const int grid = (blocks + 15) / 16;
  hipLaunchKernelGGL(quantize_q8k_kernel<true>, dim3(grid), dim3(256), 0, stream, x, a.q, a.d,
                     a.bsums, m_rows, k, nb);
}

// bfloat16 -> float32, exactly, four values per thread (n a multiple of 4, both 8-byte aligned).
__global__ __launch_bounds__(256) void widen_bf16_kernel(const uint16_t* __restrict__ x,
                                                         float* __restrict__ out, long long n4) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const uint2 h = ((const uint2*)x)[i];
  ((float4*)out)[i] = float4{bf16_to_float(h.x), bf16_to_float(h.x >> 16), bf16_to_float(h.y),
                             bf16_to_float(h.y >> 16)};
}

void launch_widen_bf16(const uint16_t* x, float* out, long long n, hipStream_t stream) {
  const long long n4 = n / 4;
  hipLaunchKernelGGL(widen_bf16_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream,
                     x, out, n4);
}

// ---------------------------------------------------------------------------------------------
// Dequantization. Each thread writes 8 consecutive values of one block (Q8_0: 4 threads per
// 32-value block; the 256-value types: 32 threads per block). Blocks come either straight from a
// flat block array, or (row gather) from whole packed rows picked by an index list; an index
// outside [0, n_src_rows) yields NaN values instead of a read.

struct DequantSrc {
  const uint8_t* base;
  const int32_t* rows;  // null: flat block array
  long long n_src_rows;
  long long row_bytes;
  int blocks_per_row;
};

template <int TYPE>
struct Geo;
template <>
struct Geo<T_Q8_0> {
  static constexpr int kElems = 32, kBytes = 34;
};
template <>
struct Geo<T_Q4_K> {
  static constexpr int kElems = 256, kBytes = 144;
};
template <>
struct Geo<T_Q6_K> {
  static constexpr int kElems = 256, kBytes = 210;
};
template <>
struct Geo<T_IQ4_XS> {
  static constexpr int kElems = 256, kBytes = 136;
};

// The 8 values of elements e0..e0+7 of one block at `blk` (byte-granular reads: the dequant
// kernels are not on the matmul path and must accept any block alignment).
template <int TYPE>
__device__ __forceinline__ void dequant8(const uint8_t* __restrict__ blk, int e0, float* v);

template <>
__device__ __forceinline__ void dequant8<T_Q8_0>(const uint8_t* __restrict__ blk, int e0, float* v) {
  const float d = half_to_float(blk[0] | (blk[1] << 8));
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)blk[2 + e0 + i] * d;
}

template <>
__device__ __forceinline__ void dequant8<T_Q4_K>(const uint8_t* __restrict__ blk, int e0, float* v) {
  // value = (d * sc) * q - (dmin * m)   (app/gguf/dequant/kquants.py:57-61)
  const float d = half_to_float(blk[0] | (blk[1] << 8));
  const float dmin = half_to_float(blk[2] | (blk[3] << 8));
  const int c = e0 >> 6, hi = (e0 >> 5) & 1, l0 = e0 & 31;
  const int j = 2 * c + hi;
  const uint8_t* s = blk + 4;
  const int sc = j < 4 ? (s[j] & 63) : ((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
  const int mn = j < 4 ? (s[j + 4] & 63) : ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  const float ds = d * (float)sc;
  const float dm = dmin * (float)mn;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint8_t byte = blk[16 + 32 * c + l0 + i];
    const int u = hi ? (byte >> 4) : (byte & 15);
    v[i] = ds * (float)u - dm;
  }
}

template <>
__device__ __forceinline__ void dequant8<T_Q6_K>(const uint8_t* __restrict__ blk, int e0, float* v) {
  // value = (d * sc) * (u - 32)   (app/gguf/dequant/kquants.py:144-159)
  const float d = half_to_float(blk[208] | (blk[209] << 8));
  const int h = e0 >> 7, g = (e0 >> 5) & 3, l0 = e0 & 31;
  const float ds = d * (float)(int8_t)blk[192 + (e0 >> 4)];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int l = l0 + i;
    const uint8_t qlb = blk[64 * h + ((g & 1) ? 32 : 0) + l];
    const int nib = (g & 2) ? (qlb >> 4) : (qlb & 15);
    const int u = nib | (((blk[128 + 32 * h + l] >> (2 * g)) & 3) << 4);
    v[i] = ds * ((float)u - 32.0f);
  }
}

template <>
__device__ __forceinline__ void dequant8<T_IQ4_XS>(const uint8_t* __restrict__ blk, int e0,
                                                   float* v) {
  // value = (d * (ls - 32)) * grid[idx]   (app/gguf/dequant/iq_ternary.py:78-89)
  const float d = half_to_float(blk[0] | (blk[1] << 8));
  const int ib = e0 >> 5, hi = (e0 >> 4) & 1, l0 = e0 & 15;
  const int sh = blk[2] | (blk[3] << 8);
  const int ls = ((blk[4 + (ib >> 1)] >> (4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
  const float dl = d * (float)(ls - 32);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint8_t byte = blk[8 + 16 * ib + l0 + i];
    const int idx = hi ? (byte >> 4) : (byte & 15);
    const uint32_t g = iq4_grid_word(idx >> 2);
    v[i] = dl * (float)(int8_t)(uint8_t)(g >> (8 * (idx & 3)));
  }
}

template <int TYPE>
__global__ __launch_bounds__(256) void dequant_kernel(DequantSrc src, long long n_blocks,
                                                      float* __restrict__ out) {
  constexpr int kThreads = Geo<TYPE>::kElems / 8;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long g = t / kThreads;
  if (g >= n_blocks) return;
  const int e0 = (int)(t - g * kThreads) * 8;
  float v[8];
  bool ok = true;
  const uint8_t* blk;
  if (src.rows != nullptr) {
    const long long r = g / src.blocks_per_row;
    const long long bi = g - r * src.blocks_per_row;
    const long long row = src.rows[r];
    ok = row >= 0 && row < src.n_src_rows;
    blk = src.base + (ok ? row : 0) * src.row_bytes + bi * Geo<TYPE>::kBytes;
  } else {
    blk = src.base + g * Geo<TYPE>::kBytes;
  }
  if (ok) {
    dequant8<TYPE>(blk, e0, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_nanf("");
  }
  float4* o = (float4*)(out + g * Geo<TYPE>::kElems + e0);
  o[0] = make_float4(v[0], v[1], v[2], v[3]);
  o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

template <int TYPE>
static void launch_dequant_t(const DequantSrc& src, long long n_blocks, float* out,
                             hipStream_t stream) {
  const long long threads = n_blocks * (Geo<TYPE>::kElems / 8);
  const long long grid = (threads + 255) / 256;
  hipLaunchKernelGGL(dequant_kernel<TYPE>, dim3((unsigned)grid), dim3(256), 0, stream, src,
                     n_blocks, out);
}

int launch_dequant(int type, const uint8_t* base, const int32_t* rows, long long n_src_rows,
                   long long row_bytes, int blocks_per_row, long long n_blocks, float* out,
                   hipStream_t stream) {
  const DequantSrc src{base, rows, n_src_rows, row_bytes, blocks_per_row};
  switch (type) {
    case T_Q8_0: launch_dequant_t<T_Q8_0>(src, n_blocks, out, stream); return 0;
    case T_Q4_K: launch_dequant_t<T_Q4_K>(src, n_blocks, out, stream); return 0;
    case T_Q6_K: launch_dequant_t<T_Q6_K>(src, n_blocks, out, stream); return 0;
    case T_IQ4_XS: launch_dequant_t<T_IQ4_XS>(src, n_blocks, out, stream); return 0;
    default: return -1;
  }
}

}  // namespace mxa
