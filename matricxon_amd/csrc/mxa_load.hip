// Load path: reordering packed rows on the device. Every GGUF type packs a row of a 2-D weight
// into whole blocks, so row i is bytes [i * row_bytes, (i + 1) * row_bytes) and rows move as
// opaque byte ranges (app/gguf/packed_rows.py:1-5). dst row i = src row order[i], the device twin
// of PackedRows.reordered (packed_rows.py:24-28), which the loader uses for the rope row
// permutation of attn_q / attn_k (app/architectures/layers.py:9-29).
//
// HBM-bound copy: each workgroup moves whole rows with the widest unit (16, 8, 4, 2 or 1 bytes)
// that divides the row and both base addresses; rows are read and written contiguously.
#include "mxa_kernels.hpp"

namespace mxa {
namespace {

constexpr int kGatherThreads = 256;

template <class U>
__global__ __launch_bounds__(kGatherThreads) void gather_rows_kernel(
    const U* __restrict__ src, long long n_src_rows, const int32_t* __restrict__ order, int n_rows,
    long long row_units, U* __restrict__ dst) {
  for (int i = blockIdx.x; i < n_rows; i += gridDim.x) {
    const long long r = order[i];
    U* d = dst + (size_t)i * row_units;
    if (r < 0 || r >= n_src_rows) {  // an index out of range gives a row of zero bytes
      for (long long c = threadIdx.x; c < row_units; c += kGatherThreads) d[c] = U{};
      continue;
    }
    const U* s = src + (size_t)r * row_units;
    for (long long c = threadIdx.x; c < row_units; c += kGatherThreads) d[c] = s[c];
  }
}

template <class U>
void launch_gather_u(const void* src, long long n_src_rows, long long row_bytes,
                     const int32_t* order, int n_rows, void* dst, hipStream_t stream) {
  const int grid = n_rows < 8192 ? n_rows : 8192;
  hipLaunchKernelGGL(gather_rows_kernel<U>, dim3(grid), dim3(kGatherThreads), 0, stream,
                     (const U*)src, n_src_rows, order, n_rows, row_bytes / (long long)sizeof(U),
                     (U*)dst);
}

}  // namespace

void launch_gather_rows(const void* src, long long n_src_rows, long long row_bytes,
                        const int32_t* order, int n_rows, void* dst, hipStream_t stream) {
  const uintptr_t a = (uintptr_t)src | (uintptr_t)dst | (uintptr_t)row_bytes;
  if ((a & 15) == 0)
    launch_gather_u<uint4>(src, n_src_rows, row_bytes, order, n_rows, dst, stream);
  else if ((a & 7) == 0)
    launch_gather_u<uint2>(src, n_src_rows, row_bytes, order, n_rows, dst, stream);
  else if ((a & 3) == 0)
    launch_gather_u<uint32_t>(src, n_src_rows, row_bytes, order, n_rows, dst, stream);
  else if ((a & 1) == 0)
    launch_gather_u<uint16_t>(src, n_src_rows, row_bytes, order, n_rows, dst, stream);
  else
    launch_gather_u<uint8_t>(src, n_src_rows, row_bytes, order, n_rows, dst, stream);
}

}  // namespace mxa
