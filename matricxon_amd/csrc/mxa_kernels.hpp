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

// Q8_K of one 256-value block held by 16 lanes of a DPP row (lane part p: its values 16p..16p+15
// in v), restating mx_quantize_row_q8_k (app/native/src/mx_common.c:42-69): amax over the block
// (fmaxf from 0: a NaN input never becomes amax, as the reference's `ax > amax ? ax : amax`); an
// all-zero block gives q = 0, bsums = 0, d = 0; otherwise iscale = 127/amax and d = amax/127 are
// correctly rounded divisions, q = clamp(round-half-even(x * iscale), +-127) (lrintf in the
// default rounding mode is v_rndne_f32), and bsums are the sums of q over 16 values. Writes the
// lane's 16 q at qblk + 16p, its bsum at bsblk[p] and, from part 0, d. All 16 lanes must be active.
__device__ __forceinline__ void q8k_part16(const float (&v)[16], int p, int8_t* qblk, int16_t* bsblk,
                                           float* dp) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = max16(amax);
  int qv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) qv[i] = 0;
  if (amax != 0.0f) {
    const float iscale = 127.0f / amax;
#pragma unroll
    for (int i = 0; i < 16; ++i) qv[i] = (int)fminf(fmaxf(rintf(v[i] * iscale), -127.0f), 127.0f);
  }
  uint32_t packed[4];
  int bsum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    packed[i] = (uint32_t)(qv[4 * i] & 0xFF) | ((uint32_t)(qv[4 * i + 1] & 0xFF) << 8) |
                ((uint32_t)(qv[4 * i + 2] & 0xFF) << 16) | ((uint32_t)(qv[4 * i + 3] & 0xFF) << 24);
    bsum += qv[4 * i] + qv[4 * i + 1] + qv[4 * i + 2] + qv[4 * i + 3];
  }
  *(uint4*)(qblk + 16 * p) = uint4{packed[0], packed[1], packed[2], packed[3]};
  bsblk[p] = (int16_t)bsum;
  if (p == 0) *dp = amax / 127.0f;
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
// The same from bfloat16 x (x widened exactly first; x 16-byte aligned).
void launch_quantize_q8k_bf16(const uint16_t* x, const ActBuffers& a, int m_rows, int k,
                              hipStream_t stream);
// out[i] = x[i] widened from bfloat16 to float32 (n a multiple of 4; x 8-, out 16-byte aligned).
void launch_widen_bf16(const uint16_t* x, float* out, long long n, hipStream_t stream);

// Fused producers: RMSNorm (mx_rms_norm, app/native/src/mx_fused_ops.c:6-17) and SwiGLU's
// silu(gate) * up (mx_silu_mul, mx_fused_ops.c:36-42) over m_rows rows of k values, writing the fp32
// result to out (when not nullptr) and its Q8_K blocks to a.
void launch_rms_norm_q8k(const float* x, const float* w, float eps, float* out, const ActBuffers& a,
                         int m_rows, int k, hipStream_t stream);
// gate and up rows are ld floats apart.
void launch_silu_mul_q8k(const float* gate, const float* up, long long ld, float* out,
                         const ActBuffers& a, int m_rows, int k, hipStream_t stream);
// The bfloat16 forms, with the reference's torch steps for a bfloat16 layer (each elementwise
// result rounded to bfloat16 as torch rounds it); Q8_K of the bfloat16 result. -1 when the rows
// are too long (RMSNorm: above 16384 values) or the operands not 8-byte aligned (ld % 4 != 0).
int launch_rms_norm_q8k_bf16(const uint16_t* x, const uint16_t* w, float eps, uint16_t* out,
                             const ActBuffers& a, int m_rows, int k, hipStream_t stream);
int launch_silu_mul_q8k_bf16(const uint16_t* gate, const uint16_t* up, long long ld, uint16_t* out,
                             const ActBuffers& a, int m_rows, int k, hipStream_t stream);

// Reads bytes (a multiple of 16) at src once and discards them; may write one word to sink.
void launch_stream_read(const void* src, long long bytes, uint32_t* sink, hipStream_t stream);

// dst row i = src row order[i] for i < n_rows (rows of row_bytes bytes); an index outside
// [0, n_src_rows) gives a zero row.
void launch_gather_rows(const void* src, long long n_src_rows, long long row_bytes,
                        const int32_t* order, int n_rows, void* dst, hipStream_t stream);


int launch_dequant(int type, const uint8_t* base, const int32_t* rows, long long n_src_rows,
                   long long row_bytes, int blocks_per_row, long long n_blocks, float* out,
                   hipStream_t stream);

// Text that mxa_last_error() returns on the calling thread until the next error.
void set_last_error(const char* text);

// Compute units of the current device (cached per device after the first call; thread-safe).
int cu_count();

// Lets `kernel` use `bytes` of dynamic LDS on the current device: the attribute is set once per
// (kernel, device, size), under a lock, so concurrent host threads may launch.
void allow_lds(const void* kernel, int bytes);

// Activation rows up to which the pipelined decode kernel takes a K-quant / Q8_0 matrix by
// default, quantizing x itself (no workspace); IQ4_XS (which reads x as floats) always takes up to
// kFusedQuantMaxRows rows there, larger decode batches in passes of that many rows.
constexpr int kDecodeMaxRows = 3;
constexpr int kFusedQuantMaxRows = 4;

// The current crossover (kDecodeMaxRows unless changed by set_fused_max_rows, clamped to
// [0, kFusedQuantMaxRows]): rows up to it take the decode kernel, more rows the matrix cores.
// Process-wide, read atomically by every launch.
int fused_max_rows();
void set_fused_max_rows(int n);

// Decode GEMV for 1 <= m_rows <= 4: y[m * ldy + n] for m < m_rows, n < n_rows (out_features) of
// one packed weight, lane-per-block compute on weight rows staged into LDS by coalesced copies. A
// K-quant or Q8_0 weight with act.q == nullptr quantizes act.x to Q8_K in the kernel.
int launch_gemv_lpb(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                    long long ldy, int m_rows, int n_rows, hipStream_t stream);

// The same GEMV on float activations (x is not quantized; the K-quants and Q8_0 take each block
// as d * sc * q - dmin * m in float against x, IQ4_XS as always): y[m * ldy + n] for
// m < m_rows <= 4, n < n_rows, from x (m_rows, k) row-major.
int launch_gemv_f32(int type, const uint8_t* w, long long row_bytes, const float* x, int k,
                    YOut y, long long ldy, int m_rows, int n_rows, hipStream_t stream);

// Decode GEMV in the read floor's shape (mxa_gemv_wave.hip): one workgroup per CU, every weight
// byte requested at once, lane-per-block compute as each wave's rows land. y[m * ldy + n] for
// m < m_rows <= 2, n < n_rows; quantizes act.x to Q8_K in the kernel when act.q == nullptr.
// Q4_K / Q8_0 / Q6_K with K / 256 in {4, 8, 16, 32, 64} (56 on workspace Q8_K; {8, 16, 32} for
// two rows), 16-byte aligned rows, and the rows per CU the type allows; -1 otherwise.
int launch_gemv_wave_m(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                       long long ldy, int m_rows, int n_rows, hipStream_t stream);
// The same for one activation row.
int launch_gemv_wave(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                     int n_rows, hipStream_t stream);
// The fp32-activation forms of Q4_K, Q6_K, Q8_0 (d * sc * q met by unquantized x) on the
// floor-shaped kernel, m_rows <= 4; -1 where it does not apply.
int launch_gemv_wave_f32(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                         long long ldy, int m_rows, int n_rows, hipStream_t stream);

// Decode GEMV for one activation row on a workgroup-resident weight share (mxa_gemv_res.hip):
// y[n] for n < n_rows. Quantizes act.x to Q8_K in the kernel when act.q == nullptr (IQ4_XS reads
// it as floats). -1 when the weight is larger than the kernel is used for, or the shape or
// alignment does not suit it.
int launch_gemv_res(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                     int n_rows, hipStream_t stream);

// One of several packed weights that share the activations of a multi-weight launch.
struct DecodeSeg {
  int type;
  const uint8_t* w;
  long long row_bytes;
  YOut y;  // the weight's first output column (row stride ldy)
  int n;     // output rows of the weight
};

// One token's routed experts in the floor-shaped kernel: pair p of n_pairs writes y + p * n_rows
// from expert ids[p] (device int32, clamped to [0, n_experts)) at w + ids[p] * expert_stride and
// activation row p * x_step (x_step 0: one row shared by all pairs). -1 when the shape does not
// suit it.
int launch_gemv_wave_pairs(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                           const int32_t* ids, int n_experts, int n_pairs, int x_step,
                           const Act& act, YOut y, int n_rows, hipStream_t stream);

// One-row decode over up to 4 Q4_K / Q6_K / Q8_0 weights sharing the activations, in the
// floor-shaped kernel (mxa_gemv_wave.hip); -1 when the weights do not suit it.
int launch_gemv_wave_multi(const DecodeSeg* seg, int count, const Act& act, hipStream_t stream);

// Decode for 1 <= m_rows <= 4 over up to 4 K-quant / Q8_0 weights in one launch (shared-input
// projections such as q/k/v or gate/up); quantizes act.x itself when act.q == nullptr. -1 when
// the weights do not suit it (the caller launches them one by one).
int launch_decode_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int m_rows,
                        hipStream_t stream);

// Matrix-core kernel for m_rows > 4 (batched decode and prefill) on Q8_K activations already in
// the workspace: Q4_K, Q6_K, Q8_0.
bool mtile_supported(int type);
int launch_mtile(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream);

// Grouped MoE projection (mxa_mtile.hip): expert e of n_experts multiplies rows
// [offsets[e], offsets[e + 1]) of the total_rows Q8_K activation rows in `act` (a device array of
// n_experts + 1 ascending offsets; at most max_rows rows per expert) by its packed weight
// w + e * expert_stride (n_rows x row_bytes), writing the same rows of y. Q4_K, Q6_K, Q8_0; -1
// otherwise.
int launch_moe_dec(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                   int n_experts, const Act& act, const int32_t* offsets, int total_rows,
                   int max_rows, YOut y, long long ldy, int n_rows, hipStream_t stream);

// The same for IQ4_XS experts on float activations act.x (the decode body, four rows at a time):
// each row equals that row multiplied alone by mxa_gemm's decode kernels. -1 otherwise.
int launch_moe_lpb(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                   int n_experts, const Act& act, const int32_t* offsets, int total_rows,
                   int max_rows, YOut y, long long ldy, int n_rows, hipStream_t stream);

// out[t] (n_tokens x n_embd fp32) = the routing-weighted sum of token t's expert outputs:
// down row rows[t top_k + k] (rows == nullptr: row t top_k + k) of slot k, times weights[t top_k
// + k], slots in ascending ids[t top_k + k] (ties in slot order), bf16 != 0: each down value
// rounded to bfloat16 first. top_k <= kMoeMaxTopK; -1 otherwise.
constexpr int kMoeMaxTopK = 16;
// MoE routing (one workgroup, stable counting sort): up to kMoeRouteMaxExperts experts and
// kMoeRouteMaxPairs (token, slot) pairs; -1 otherwise.
constexpr int kMoeRouteMaxExperts = 256;
constexpr int kMoeRouteMaxPairs = 1 << 20;
int launch_moe_route(const void* ids, bool ids64, int n_tokens, int top_k, int n_experts,
                     int32_t* offsets, int32_t* pair_tok, int32_t* rows, int32_t* ids32,
                     hipStream_t stream);
int launch_moe_combine(const float* down, const int32_t* rows, const int32_t* ids,
                       const float* weights, int n_tokens, int top_k, int n_embd, int bf16,
                       float* out, hipStream_t stream);

// Batched decode (m_rows <= 16) on the matrix cores with the weight rows streamed into LDS by
// coalesced copies, one persistent workgroup per CU: Q4_K, Q6_K, Q8_0 on Q8_K activations in the
// workspace. -1 when the shape does not suit it (the caller uses launch_mtile).
int launch_bstream(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                   long long ldy, int m_rows, int n_rows, hipStream_t stream);

// Batched decode (m_rows <= 16, rows of up to 16 blocks) in which every wave gathers, computes
// and (the last of each tile) folds its own block columns (mxa_bwave.hip): Q4_K, Q6_K, Q8_0 on
// Q8_K activations in the workspace, 16-byte aligned weight and rows. -1 when the workgroup's
// slots do not fit LDS.
int launch_bwave(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream);
// Shared-input K-quant weights (2..4, Q4_K / Q6_K, rows of up to 16 blocks, each resident) at
// 1..16 activation rows on Q8_K blocks in one launch of the gather kernel; -1 when it does not
// take the group.
int launch_bwave_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int m_rows,
                       hipStream_t stream);
// Grouped MoE experts on the batched-decode bodies (short and long rows): rows
// [offsets[e], offsets[e + 1]) of the Q8_K activations through the expert at w + e *
// expert_stride, in 16-row passes; -1 when the geometry does not fit (the caller takes another
// grouped form).
int launch_moe_bwave(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                     int n_experts, const Act& act, const int32_t* offsets, int total_rows,
                     YOut y, long long ldy, int n_rows, hipStream_t stream);

// Batched decode (m_rows <= 16, rows of up to 16 blocks) with the workgroup's whole weight share
// resident in LDS, streamed in by copy waves while compute waves run the matrix cores
// (mxa_bflow.hip): Q4_K, Q6_K, Q8_0 on Q8_K activations in the workspace, 16-byte aligned weight
// and rows. -1 when the share does not fit LDS (the caller uses launch_bres).
int launch_bflow(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream);

// Batched decode (m_rows <= 16, rows of up to 16 blocks) with each workgroup's weight rows
// streamed through LDS in 16-row tiles, in order: Q4_K, Q6_K, Q8_0 on Q8_K activations in the
// workspace. -1 when the geometry does not fit (the caller uses launch_bstream).
int launch_bres(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
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
                       YOut y, long long ldy, int m_rows, int k, int n_rows, hipStream_t stream);

// The matmul for any m_rows: picks the kernel (mxa_dispatch.hip); -1 when no kernel applies.
int launch_matmul(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                  long long ldy, int m_rows, int n_rows, hipStream_t stream);

}  // namespace mxa
