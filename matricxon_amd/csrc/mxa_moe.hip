// Weighted combine of routed expert outputs (MoE), one launch: for token t, the down-projection
// rows of its top_k (token, slot) pairs times the routing weights, summed in ascending expert id
// (pairs of equal id in slot order) from a float zero, as the reference's loop over the sorted
// expert ids adds them with `index_add_` (app/architectures/moe_experts.py:81-88), with the
// module's casts: the projection output rounded to bfloat16 first when the layer computes in
// bfloat16 (`down.to(dtype)`), the product with the float32 weight rounded to float32, each sum
// rounded to float32. One thread per output element; the pair order is ranked once per workgroup.
#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

// float32 -> bfloat16 -> float32 with round-to-nearest-even, NaN to the quiet NaN 0x7FC0 (the
// conversion torch's `.to(torch.bfloat16)` performs)
__device__ __forceinline__ float round_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float(0x7FC00000u);
  return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}

__global__ __launch_bounds__(256) void moe_combine_kernel(
    const float* __restrict__ down, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ ids, const float* __restrict__ wts, int top_k, int n_embd,
    int bf16, float* __restrict__ out) {
  __shared__ int ord[kMoeMaxTopK];
  const int t = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
  const int32_t* tid = ids + (size_t)t * top_k;
  if ((int)threadIdx.x < top_k) {  // slot k's place in the token's sorted order
    const int k = threadIdx.x, e = tid[k];
    int rank = 0;
    for (int k2 = 0; k2 < top_k; ++k2) rank += (tid[k2] < e) || (tid[k2] == e && k2 < k);
    ord[rank] = k;
  }
  __syncthreads();
  if (j >= n_embd) return;
  float acc = 0.0f;
  for (int i = 0; i < top_k; ++i) {
    const size_t p = (size_t)t * top_k + ord[i];
    const size_t r = rows != nullptr ? (size_t)rows[p] : p;
    float v = down[r * n_embd + j];
    if (bf16) v = round_bf16(v);
    acc = acc + v * wts[p];
  }
  out[(size_t)t * n_embd + j] = acc;
}

}  // namespace

int launch_moe_combine(const float* down, const int32_t* rows, const int32_t* ids,
                       const float* weights, int n_tokens, int top_k, int n_embd, int bf16,
                       float* out, hipStream_t stream) {
  if (n_tokens < 1 || n_tokens > 65535 || top_k < 1 || top_k > kMoeMaxTopK || n_embd < 1)
    return -1;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((n_embd + 255) / 256, n_tokens), dim3(256), 0,
                     stream, down, rows, ids, weights, top_k, n_embd, bf16, out);
  return 0;
}

}  // namespace mxa
