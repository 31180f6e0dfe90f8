// Host-visible kernel launchers shared between the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mxa_device.hpp"

namespace mxa {

// Device layout of the Q8_K activations inside the caller's workspace (each part 256-B aligned):
// q int8 (M, K) | d float (M, K/256) | bsums int16 (M, K/256, 16).
struct ActBuffers {
  int8_t* q;
  float* d;
  int16_t* bsums;
};

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

inline size_t act_bytes(int m_rows, int k) {
  const size_t nb = (size_t)k / QK;
  return align256((size_t)m_rows * k) + align256((size_t)m_rows * nb * 4) +
         align256((size_t)m_rows * nb * 16 * 2);
}

inline ActBuffers act_layout(void* ws, int m_rows, int k) {
  const size_t nb = (size_t)k / QK;
  uint8_t* p = (uint8_t*)ws;
  ActBuffers a;
  a.q = (int8_t*)p;
  p += align256((size_t)m_rows * k);
  a.d = (float*)p;
  p += align256((size_t)m_rows * nb * 4);
  a.bsums = (int16_t*)p;
  return a;
}

void launch_quantize_q8k(const float* x, const ActBuffers& a, int m_rows, int k,
                         hipStream_t stream);


int launch_dequant(int type, const uint8_t* base, const int32_t* rows, long long n_src_rows,
                   long long row_bytes, int blocks_per_row, long long n_blocks, float* out,
                   hipStream_t stream);

// Compute units of the current device (cached after the first call).
int cu_count();

// Activation rows up to which the pipelined decode kernel takes a matrix, quantizing x itself (no
// workspace): K-quant / Q8_0 weights, and IQ4_XS (which reads x as floats; larger decode batches
// run in passes of this many rows).
constexpr int kDecodeMaxRows = 3;
constexpr int kFusedQuantMaxRows = 4;

// Decode GEMV for 1 <= m_rows <= 4: y[m * ldy + n] for m < m_rows, n < n_rows (out_features) of
// one packed weight, lane-per-block compute on weight rows staged into LDS by coalesced copies. A
// K-quant or Q8_0 weight with act.q == nullptr quantizes act.x to Q8_K in the kernel.
int launch_gemv_lpb(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                    long long ldy, int m_rows, int n_rows, hipStream_t stream);

// One of several packed weights that share the activations of a multi-weight launch.
struct DecodeSeg {
  int type;
  const uint8_t* w;
  long long row_bytes;
  float* y;  // the weight's first output column (row stride ldy)
  int n;     // output rows of the weight
};

// Decode for 1 <= m_rows <= 4 over up to 4 K-quant / Q8_0 weights in one launch (shared-input
// projections such as q/k/v or gate/up); quantizes act.x itself when act.q == nullptr. -1 when
// the weights do not suit it (the caller launches them one by one).
int launch_decode_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int m_rows,
                        hipStream_t stream);

// Matrix-core kernel for m_rows > 4 (batched decode and prefill) on Q8_K activations already in
// the workspace: Q4_K, Q6_K, Q8_0.
bool mtile_supported(int type);
int launch_mtile(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream);

// Batched decode (m_rows <= 16) on the matrix cores with the weight rows streamed into LDS by
// coalesced copies, one persistent workgroup per CU: Q4_K, Q6_K, Q8_0 on Q8_K activations in the
// workspace. -1 when the shape does not suit it (the caller uses launch_mtile).
int launch_bstream(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                   long long ldy, int m_rows, int n_rows, hipStream_t stream);

// Batched decode (m_rows <= 16, rows of up to 16 blocks) with each workgroup's weight rows
// streamed through LDS in 16-row tiles, in order: Q4_K, Q6_K, Q8_0 on Q8_K activations in the
// workspace. -1 when the geometry does not fit (the caller uses launch_bstream).
int launch_bres(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                long long ldy, int m_rows, int n_rows, hipStream_t stream);
// The same over up to 4 weights sharing the activations, in one launch.
int launch_bres_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int m_rows,
                      hipStream_t stream);

// The streaming batched decode over up to 4 K-quant / Q8_0 weights that share the activations,
// in one launch. -1 when the weights do not suit it.
int launch_bstream_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int m_rows,
                         hipStream_t stream);

// IQ4_XS prefill on the matrix cores (m_rows >= kIq4MfmaMinRows): x split into bf16 hi / lo in
// `workspace` (iq4_prefill_workspace bytes), then bf16 MFMAs per 32-value sub-block.
constexpr int kIq4MfmaMinRows = 17;
size_t iq4_prefill_workspace(int m_rows, int k);
int launch_iq4_prefill(const uint8_t* w, long long row_bytes, const float* x, void* workspace,
                       float* y, long long ldy, int m_rows, int k, int n_rows, hipStream_t stream);

// The matmul for any m_rows: picks the kernel (mxa_dispatch.hip); -1 when no kernel applies.
int launch_matmul(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                  long long ldy, int m_rows, int n_rows, hipStream_t stream);

}  // namespace mxa
