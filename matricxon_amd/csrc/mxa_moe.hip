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

// Routing of the (token, slot) pairs by expert, one workgroup: a stable counting sort. Pair
// p = t * top_k + k has expert e = ids[p] clamped into [0, n_experts); its place in the sorted
// order is the pairs of smaller experts plus the earlier pairs of the same expert, which is where
// a stable argsort of the flattened ids puts it (the order the reference's per-expert loop visits
// tokens: moe_experts.py:81-88, tokens ascending within an expert). Histogram (LDS atomics),
// exclusive scan over experts, then chunks of 1024 pairs in order: each wave ranks its lanes
// among equal experts with ballots, the waves' counts are prefixed per expert, and a per-expert
// base carries from chunk to chunk.
constexpr int kRouteWaves = 16;
__global__ __launch_bounds__(64 * kRouteWaves) void moe_route_kernel(
    const void* __restrict__ ids, int ids64, int n_pairs, int top_k, int n_experts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ pair_tok, int32_t* __restrict__ rows,
    int32_t* __restrict__ ids32) {
  __shared__ int cnt[kMoeRouteMaxExperts];
  __shared__ int scan[2][kMoeRouteMaxExperts];
  __shared__ int base[kMoeRouteMaxExperts];
  __shared__ int wcnt[kRouteWaves][kMoeRouteMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  auto raw = [&](int p) -> long long {
    return ids64 ? ((const long long*)ids)[p] : (long long)((const int32_t*)ids)[p];
  };
  auto expert = [&](long long v) { return v < 0 ? 0 : v >= n_experts ? n_experts - 1 : (int)v; };
  if (tid < kMoeRouteMaxExperts) cnt[tid] = 0;
  __syncthreads();
  for (int p = tid; p < n_pairs; p += 64 * kRouteWaves) {
    const long long v = raw(p);
    atomicAdd(&cnt[expert(v)], 1);
    if (ids32 != nullptr) ids32[p] = (int32_t)v;  // torch's int64 -> int32 conversion
  }
  __syncthreads();
  // inclusive scan of the counts (Hillis-Steele over kMoeRouteMaxExperts entries)
  int cur = 0;
  if (tid < kMoeRouteMaxExperts) scan[0][tid] = tid < n_experts ? cnt[tid] : 0;
  for (int off = 1; off < kMoeRouteMaxExperts; off <<= 1) {
    __syncthreads();
    if (tid < kMoeRouteMaxExperts) {
      int x = scan[cur][tid];
      if (tid >= off) x += scan[cur][tid - off];
      scan[cur ^ 1][tid] = x;
    }
    cur ^= 1;
  }
  __syncthreads();
  if (tid < n_experts) {
    base[tid] = scan[cur][tid] - cnt[tid];
    offsets[tid] = base[tid];
  }
  if (tid == 0) offsets[n_experts] = n_pairs;
  for (int c0 = 0; c0 < n_pairs; c0 += 64 * kRouteWaves) {
    for (int i = tid; i < kRouteWaves * kMoeRouteMaxExperts; i += 64 * kRouteWaves)
      wcnt[i / kMoeRouteMaxExperts][i % kMoeRouteMaxExperts] = 0;
    __syncthreads();  // also: base is set (first chunk) or carried (later chunks)
    const int p = c0 + tid;
    const bool valid = p < n_pairs;
    const int e = valid ? expert(raw(p)) : -1;
    int rank = 0;  // earlier lanes of this wave with the same expert
    uint64_t rem = __ballot(valid);
    while (rem != 0) {  // wave-uniform: one pass per distinct expert of the wave
      const int leader = __builtin_ctzll(rem);
      const int v = __builtin_amdgcn_readlane(e, leader);
      const uint64_t m = __ballot(valid && e == v);
      if (valid && e == v) rank = __popcll(m & ((1ull << lane) - 1ull));
      if (lane == 0) wcnt[wave][v] = __popcll(m);
      rem &= ~m;
    }
    __syncthreads();
    if (tid < n_experts) {  // the waves' counts prefixed per expert, from the carried base
      int run = base[tid];
      for (int w = 0; w < kRouteWaves; ++w) {
        const int t = wcnt[w][tid];
        wcnt[w][tid] = run;
        run += t;
      }
      base[tid] = run;
    }
    __syncthreads();
    if (valid) {
      const int sidx = wcnt[wave][e] + rank;
      rows[p] = sidx;
      pair_tok[sidx] = p / top_k;
    }
    __syncthreads();  // every lane has read wcnt before the next chunk clears it
  }
}

}  // namespace

int launch_moe_route(const void* ids, bool ids64, int n_tokens, int top_k, int n_experts,
                     int32_t* offsets, int32_t* pair_tok, int32_t* rows, int32_t* ids32,
                     hipStream_t stream) {
  if (ids == nullptr || offsets == nullptr || pair_tok == nullptr || rows == nullptr ||
      n_tokens < 1 || top_k < 1 || n_experts < 1 || n_experts > kMoeRouteMaxExperts ||
      (long long)n_tokens * top_k > kMoeRouteMaxPairs)
    return -1;
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(64 * kRouteWaves), 0, stream, ids,
                     ids64 ? 1 : 0, n_tokens * top_k, top_k, n_experts, offsets, pair_tok, rows,
                     ids32);
  return 0;
}

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
