/*
 * matricxon_amd: quantized-native matmul over packed GGUF blocks on AMD Instinct MI355X (gfx950).
 *
 * C ABI of libmatricxon_amd.so. Plain pointers and sizes only. All array pointers are DEVICE
 * pointers (HBM) unless stated otherwise; `stream` is a hipStream_t (NULL = the null stream).
 * Every call is asynchronous on `stream`, keeps no pointer after it returns and allocates no
 * device memory: scratch space is the caller's `workspace`.
 *
 * Alignment: packed weights start on a 4-byte boundary; float activations `x` and `workspace`
 * on a 16-byte boundary (every allocation of the HIP allocator is); otherwise -1.
 *
 * Status codes (the reference's convention, app/native/src/mx_gemm.c:123-124, extended):
 *   0  ok
 *  -1  unsupported type or shape (the caller keeps another path; app/native/gemm.py:94-103)
 *  -2  workspace missing or too small (the reference's "out of memory")
 *  -3  kernel launch error (the HIP error string is available from mxa_last_error())
 *
 * GGML type ids (app/gguf/constants.py:24-59): Q8_0 = 8, Q4_K = 12, Q6_K = 14, IQ4_XS = 23.
 */
#ifndef MATRICXON_AMD_H
#define MATRICXON_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXA_TYPE_Q8_0 8
#define MXA_TYPE_Q4_K 12
#define MXA_TYPE_Q6_K 14
#define MXA_TYPE_IQ4_XS 23

#define MXA_OK 0
#define MXA_ERR_UNSUPPORTED (-1)
#define MXA_ERR_WORKSPACE (-2)
#define MXA_ERR_LAUNCH (-3)

/* Build description for the startup log.
 * Replaces `mx_build_info` (app/native/src/mx_gemm.c:196-220). Host-only, no GPU call. */
const char *mxa_build_info(void);

/* 1 when mxa_gemm handles (ggml_type, in_features): one of the four types and in_features a
 * positive multiple of 256; 0 otherwise.
 * Replaces `mx_supports` (app/native/src/mx_gemm.c:114-121). Host-only. */
int mxa_supports(int ggml_type, int in_features);

/* 1 when mxa_dequant_rows handles (ggml_type, row_width): one of the four types and row_width a
 * positive multiple of 256; 0 otherwise. (The reference's row dequantizer covers only the K-quants
 * with an unpack routine; this one covers all four types here.)
 * Replaces `mx_supports_dequant_rows` (app/native/src/mx_dequant_rows.c:49-56). Host-only. */
int mxa_supports_dequant_rows(int ggml_type, int row_width);

/* Activation rows up to which mxa_gemm / mxa_gemm_multi run a K-quant or Q8_0 weight on the decode
 * kernel, which quantizes x itself (no workspace); larger calls quantize into the workspace and run
 * on the matrix cores. Default 3, clamped to [0, 4]. Both kernels give the same bits, so this only
 * moves the speed crossover. Process-wide; mxa_workspace_bytes follows it, so query workspace
 * sizes after changing it.
 * Replaces `mx_set_fused_max_tokens` (app/native/src/mx_gemm.c:11-16), the reference's crossover
 * between its fused per-token kernel and the unpack-once path. Host-only. */
void mxa_set_fused_max_tokens(int n_tokens);

/* The current value of that crossover. No counterpart in the reference (its value is write-only
 * there). Host-only. */
int mxa_fused_max_tokens(void);

/* Bytes of one packed row of `in_features` values (0 when unsupported). Host-only. */
size_t mxa_row_bytes(int ggml_type, int in_features);

/* Workspace bytes mxa_gemm needs for n_tokens rows of in_features. Q8_0 / Q4_K / Q6_K: the Q8_K
 * activation blocks, or 0 for up to 3 rows (the matmul kernel quantizes them in on-chip memory
 * itself). IQ4_XS: 0 for up to 16 rows; from 17 rows (prefill on the matrix cores) the bf16
 * hi / lo split of x, 4 * n_tokens * in_features bytes. mxa_gemm_multi over both kinds needs the
 * sum of the largest of each kind. Host-only. */
size_t mxa_workspace_bytes(int ggml_type, int n_tokens, int in_features);

/* y (n_tokens, out_features) fp32 = x (n_tokens, in_features) fp32 @ W.T, W the packed rows
 * (out_features, row_bytes) in GGUF order. The activations are quantized to Q8_K exactly as the
 * reference C kernel does (except IQ4_XS, which uses them as floats): into `workspace` first,
 * or, for n_tokens <= 3, inside the matmul kernel (one launch, no workspace).
 * Replaces `mx_gemm` (app/native/src/mx_gemm.c:123-194) and, on the GPU, the dequantize +
 * F.linear of `DevicePackedLinear.forward` (app/architectures/device_packed.py:53-63). */
int mxa_gemm(int ggml_type, const void *w, const float *x, float *y, int n_tokens,
             int out_features, int in_features, void *workspace, size_t workspace_bytes,
             void *stream);

/* ---------------------------------------------------------------------------------------------
 * bfloat16 activations and outputs. The reference's packed GPU module computes in its layer dtype,
 * bfloat16 on a GPU (app/runtime/compute_device.py:74-78; app/architectures/device_packed.py:53-63:
 * x.to(dtype), then F.linear in that dtype). These entry points take bfloat16 x (16-byte aligned)
 * and write bfloat16 y (2-byte aligned), each output the float32 result of the float32 entry point
 * on the widened x, rounded to nearest even (NaN -> 0x7FC0), as torch's float -> bfloat16 cast
 * rounds it. No counterpart in the reference's C library (its native kernels are CPU float32). */

/* Workspace bytes of the _bf16 entry points: Q8_0 / Q4_K / Q6_K the Q8_K activations for every
 * n_tokens (x is quantized into them whenever the decode kernel that reads bfloat16 x itself does
 * not take the call); IQ4_XS x widened to float32 (4 * n_tokens * in_features bytes) plus, from 17
 * rows, the prefill split (mxa_workspace_bytes). mxa_gemm_multi_bf16 over both kinds needs the sum
 * of the largest of each kind. Host-only. */
size_t mxa_workspace_bytes_bf16(int ggml_type, int n_tokens, int in_features);

/* mxa_gemm on bfloat16 x, writing bfloat16 y. A call that the decode kernel reading bfloat16 x
 * takes (K-quant or Q8_0 weights, n_tokens <= mxa_fused_max_tokens, a supported geometry) uses no
 * workspace, so `workspace` may be NULL there; any other call with a workspace short of
 * mxa_workspace_bytes_bf16 returns MXA_ERR_WORKSPACE having launched nothing. The same holds for
 * mxa_gemm_multi_bf16 at one token. */
int mxa_gemm_bf16(int ggml_type, const void *w, const void *x, void *y, int n_tokens,
                  int out_features, int in_features, void *workspace, size_t workspace_bytes,
                  void *stream);

/* mxa_gemm_multi on bfloat16 x, writing bfloat16 y (n_tokens, sum outs). */
int mxa_gemm_multi_bf16(int n, const int *types, const void *const *ws, const int *outs,
                        const void *x, void *y, int n_tokens, int in_features, void *workspace,
                        size_t workspace_bytes, void *stream);

/* mxa_gemm_q8k writing bfloat16 y (K-quant and Q8_0 weights: the Q8_K activations are all the
 * input). */
int mxa_gemm_q8k_bf16(int ggml_type, const void *w, void *y, int n_tokens, int out_features,
                      int in_features, const void *workspace, size_t workspace_bytes,
                      void *stream);

/* mxa_gemm_multi_q8k writing bfloat16 y. */
int mxa_gemm_multi_q8k_bf16(int n, const int *types, const void *const *ws, const int *outs,
                            void *y, int n_tokens, int in_features, const void *workspace,
                            size_t workspace_bytes, void *stream);

/* mxa_quantize_q8_k of bfloat16 x (the values widened exactly). */
int mxa_quantize_q8_k_bf16(const void *x, int n_tokens, int in_features, void *workspace,
                           size_t workspace_bytes, void *stream);

/* RMSNorm of a bfloat16 layer with the steps of the reference's torch forward for bfloat16 x and
 * weight (app/architectures/layers.py:77-81): x widened to float32, variance = the mean of x^2,
 * out = bf16(bf16(x * rsqrt(variance + eps)) * weight), written to out (bfloat16, may be NULL) and
 * its Q8_K blocks to the workspace (mxa_quantize_q8_k's layout). dim <= 16384; x, weight and out
 * 8-byte aligned; else -1. The fused RMSNorm that `FusedOps.rms_norm` provides on the CPU
 * (app/native/fused_ops.py:152-158), for the GPU's bfloat16 layers. */
int mxa_rms_norm_q8_k_bf16(const void *x, const void *weight, float eps, int n_tokens, int dim,
                           void *out, void *workspace, size_t workspace_bytes, void *stream);

/* silu(gate) * up of a bfloat16 layer with torch's steps for bfloat16 tensors
 * (app/architectures/layers.py:53-57: F.silu(gate) * up): out = bf16(bf16(g / (1 + expf(-g))) *
 * u), written to out (bfloat16, contiguous, may be NULL) and its Q8_K blocks to the workspace.
 * gate and up rows are ld >= dim values apart (ld % 4 == 0; operands 8-byte aligned; else -1). */
int mxa_silu_mul_q8_k_bf16(const void *gate, const void *up, long long ld, int n_tokens, int dim,
                           void *out, void *workspace, size_t workspace_bytes, void *stream);

/* y (n_tokens, out_features) = x @ W.T with x kept in float32 (never quantized to Q8_K): each
 * weight value is its dequantized float (d * sc * q - dmin * m) meeting an unquantized activation,
 * the numerics of the reference's fp32-activation GEMV backend. Decode-sized calls: the
 * activation rows go through the kernel four at a time. No workspace. x must be 16-byte aligned.
 * Replaces the Numba GEMVs `qgemv_q4_k` (app/gguf/dequant/quantized_gemv.py:51-112),
 * `qgemv_q6_k` (quantized_gemv.py:115-180), `qgemv_q8_0`
 * (app/gguf/dequant/quantized_gemv_legacy.py:167-194) and `qgemv_iq4_xs`
 * (app/gguf/dequant/quantized_gemv_iq_ternary.py:65-107), which take one row (n_tokens == 1). */
int mxa_gemv_f32(int ggml_type, const void *w, const float *x, float *y, int n_tokens,
                 int out_features, int in_features, void *stream);

/* Bytes of the static scratch array behind mxa_gemm_static (one per device). */
#define MXA_STATIC_SCRATCH_BYTES ((size_t)16 << 20)

/* mxa_gemm with no workspace argument and no device allocation anywhere on its path, for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * it). No counterpart in the reference, whose mx_gemm mallocs its scratch per call. The first call
 * on a device does that device's set-up (the array's address, kernel attributes) and must not be
 * under graph capture; calls after one eager call of the same shape may be captured. The workspace
 * mxa_gemm would take (mxa_workspace_bytes) is a file-scope device array of
 * MXA_STATIC_SCRATCH_BYTES per device, kept until the process ends; a call that needs more
 * returns -2. Calls on one device share that array: calls that overlap on one device (other
 * streams, other host threads) race and must be ordered by the caller. */
int mxa_gemm_static(int ggml_type, const void *w, const float *x, float *y, int n_tokens,
                    int out_features, int in_features, void *stream);

/* mxa_gemm without its first step: `workspace` already holds the Q8_K activations of x
 * (written by mxa_quantize_q8_k for the same n_tokens and in_features), so only the matmul
 * kernel runs. `x` is read only for IQ4_XS (float activations) and may be NULL otherwise.
 * The reference has no separate entry: this is the second half of `mx_gemm`
 * (app/native/src/mx_gemm.c:158-190), for callers that quantize once for several weights. */
int mxa_gemm_q8k(int ggml_type, const void *w, const float *x, float *y, int n_tokens,
                 int out_features, int in_features, const void *workspace,
                 size_t workspace_bytes, void *stream);

/* Grouped projection of packed MoE experts, one launch for all of them: expert e of n_experts
 * (packed weight w + e * expert_stride bytes, out_features x row bytes; w 4-byte aligned,
 * expert_stride a multiple of 4) multiplies
 * rows [offsets[e], offsets[e + 1]) of x (n_rows, in_features) fp32, writing the same rows of
 * y (n_rows, out_features). `offsets` is a DEVICE int32 array of n_experts + 1 ascending values
 * from 0 to n_rows (the rows grouped by expert), so routing needs no host sync;
 * max_rows_per_expert picks the launch's form (the rows an expert usually has, e.g. n_tokens);
 * an expert with more rows is still computed whole, in more chunks. x == NULL:
 * `workspace` already holds the Q8_K activations of the n_rows rows (mxa_quantize_q8_k,
 * mxa_silu_mul_q8_k). workspace: mxa_quantize_q8_k's layout for n_rows rows. Each row equals
 * mxa_gemm of that row alone bit for bit. Q4_K, Q6_K, Q8_0; IQ4_XS multiplies the float rows of x
 * (x required, no workspace) with the decode kernels' arithmetic, so each row equals mxa_gemm of
 * that row alone, and an expert's rows equal mxa_gemm of them together while it has up to 16
 * (from 17 rows mxa_gemm takes the matrix cores: within the bound stated there).
 * Replaces the per-expert loop of `QuantizedMoEExperts.forward`
 * (app/architectures/moe_experts.py:81-88: one `DevicePackedLinear` call per active expert and
 * projection, after a host sync on the routed expert ids). */
int mxa_gemm_moe(int ggml_type, const void *w, long long expert_stride, int n_experts,
                 const float *x, const int32_t *offsets, int n_rows, int max_rows_per_expert,
                 float *y, int out_features, int in_features, void *workspace,
                 size_t workspace_bytes, void *stream);

/* mxa_gemm_moe writing bfloat16 y (2-byte aligned): each output the float32 result rounded to
 * nearest even as torch's cast rounds it, so the layer's bfloat16 gate and up projections need no
 * separate cast launch. No counterpart in the reference's C library: its MoE experts on the GPU
 * run in the layer's bfloat16 (app/architectures/moe_experts.py:81-88 through
 * device_packed.py:53-63). */
int mxa_gemm_moe_bf16(int ggml_type, const void *w, long long expert_stride, int n_experts,
                      const float *x, const int32_t *offsets, int n_rows, int max_rows_per_expert,
                      void *y, int out_features, int in_features, void *workspace,
                      size_t workspace_bytes, void *stream);

/* One token's routed experts (MoE decode), one launch: pair p of n_pairs multiplies expert
 * ids[p] (a DEVICE int32 array; ids outside [0, n_experts) are clamped) at w + ids[p] *
 * expert_stride (out_features x row bytes) by activation row p of x (x_rows == n_pairs) or by the
 * one row they share (x_rows == 1), writing row p of y (n_pairs, out_features). x == NULL:
 * `workspace` already holds the Q8_K activations of the x_rows rows; else x is quantized in the
 * kernel, or first into `workspace` (mxa_quantize_q8_k's layout for x_rows rows) for shapes that
 * need it. Each row equals mxa_gemm of that row alone bit for bit. Q4_K, Q6_K, Q8_0 with
 * in_features / 256 in {4, 8, 16, 32, 56, 64}, 16-byte aligned rows and expert_stride; -1 for
 * other shapes (the caller uses mxa_gemm_moe). Replaces the per-expert calls of
 * `QuantizedMoEExperts.forward` for one token (app/architectures/moe_experts.py:81-88). */
int mxa_gemm_moe_pairs(int ggml_type, const void *w, long long expert_stride, int n_experts,
                       const int32_t *ids, int n_pairs, const float *x, int x_rows, float *y,
                       int out_features, int in_features, void *workspace,
                       size_t workspace_bytes, void *stream);

/* mxa_gemm_moe_pairs on bfloat16 x (16-byte aligned; NULL: the workspace holds the Q8_K blocks
 * of the x_rows rows, as a producer such as mxa_silu_mul_q8_k_bf16 writes them), writing bfloat16
 * y (2-byte aligned): each output the float32 result rounded to nearest even as torch's cast
 * rounds it. No counterpart in the reference's C library: its MoE experts on the GPU run in the
 * layer's bfloat16 (app/architectures/moe_experts.py:81-88 through device_packed.py:53-63). */
int mxa_gemm_moe_pairs_bf16(int ggml_type, const void *w, long long expert_stride, int n_experts,
                            const int32_t *ids, int n_pairs, const void *x, int x_rows, void *y,
                            int out_features, int in_features, void *workspace,
                            size_t workspace_bytes, void *stream);

/* Routing of MoE (token, slot) pairs by expert, one launch and no host sync: ids (n_tokens,
 * top_k) DEVICE expert ids, int32 (ids_int64 = 0) or int64 (1), clamped into [0, n_experts).
 * Writes DEVICE int32 arrays: offsets (n_experts + 1; offsets[e] = the pairs of experts below e),
 * pair_tok (n_tokens * top_k: the token of each pair in expert order, tokens ascending within an
 * expert: a stable sort), rows (n_tokens * top_k: the place of pair t * top_k + k in that order)
 * and, unless NULL, ids32 (the ids converted to int32 as torch converts them). n_experts <= 256
 * and n_tokens * top_k <= 2^20, else -1. The routing of `QuantizedMoEExperts.forward`
 * (app/architectures/moe_experts.py:81-88: `top_k_idx.unique().tolist()`, then the tokens of each
 * expert by `(top_k_idx == e).nonzero()`), as the grouped launches and the combine take it. */
int mxa_moe_route(const void *ids, int ids_int64, int n_tokens, int top_k, int n_experts,
                  int32_t *offsets, int32_t *pair_tok, int32_t *rows, int32_t *ids32,
                  void *stream);

/* Routing-weighted combine of MoE expert outputs, one launch: out (n_tokens, n_embd) fp32, row t =
 * the sum over token t's top_k slots k, in ascending expert id ids[t * top_k + k] (a DEVICE int32
 * array; equal ids in slot order), of down[r] * weights[t * top_k + k] with r = rows[t * top_k +
 * k] (a DEVICE int32 array of down rows; NULL: r = t * top_k + k), from a float zero, each
 * product and sum rounded to float32. round_bf16 != 0 rounds each down value to bfloat16 first.
 * down (rows, n_embd) fp32 and weights fp32 are device arrays; top_k <= 16 (else -1). The
 * combine of `QuantizedMoEExperts.forward` (app/architectures/moe_experts.py:81-88: the
 * projection output cast to the layer dtype, times the float32 weight, `index_add_`ed into a
 * float32 zero tensor expert by expert in ascending id), bit for bit. */
int mxa_moe_combine(const float *down, const int32_t *rows, const int32_t *ids,
                    const float *weights, int n_tokens, int top_k, int n_embd, int round_bf16,
                    float *out, void *stream);

/* Up to 4 packed weights sharing one input (q/k/v, gate/up): one activation quantization, then
 * each weight's output columns written after the previous weight's, y (n_tokens, sum outs).
 * `types`, `ws` (device pointers) and `outs` are HOST arrays of n entries.
 * Replaces `mx_gemm_multi` (app/native/src/mx_gemm_multi.c:8-62); unlike the reference it
 * also accepts prefill-sized n_tokens (the reference returns -1 there). */
int mxa_gemm_multi(int n, const int *types, const void *const *ws, const int *outs,
                   const float *x, float *y, int n_tokens, int in_features, void *workspace,
                   size_t workspace_bytes, void *stream);

/* mxa_gemm_multi without its quantization step: `workspace` already holds the Q8_K activations
 * (mxa_quantize_q8_k, mxa_rms_norm_q8_k or mxa_silu_mul_q8_k for the same n_tokens and
 * in_features). K-quant and Q8_0 weights only (IQ4_XS reads float activations).
 * The second half of `mx_gemm_multi` (app/native/src/mx_gemm_multi.c:8-62), for groups whose
 * input comes from a fused producer. */
int mxa_gemm_multi_q8k(int n, const int *types, const void *const *ws, const int *outs, float *y,
                       int n_tokens, int in_features, const void *workspace,
                       size_t workspace_bytes, void *stream);

/* RMSNorm of x (n_tokens, dim) with weight (dim) and eps, as `mx_rms_norm`
 * (app/native/src/mx_fused_ops.c:6-17): out = x * (1 / sqrtf(mean(x^2) + eps)) * weight, written
 * to out (fp32, may be NULL) and, in the same pass, quantized to Q8_K into the workspace (layout of
 * mxa_quantize_q8_k; the blocks equal those of quantizing out). Replaces `FusedOps.rms_norm`
 * (app/architectures/layers.py:72-76) followed by the projections' quantization step. */
int mxa_rms_norm_q8_k(const float *x, const float *weight, float eps, int n_tokens, int dim,
                      float *out, void *workspace, size_t workspace_bytes, void *stream);

/* SwiGLU's middle step out = silu(gate) * up = gate / (1 + expf(-gate)) * up, elementwise over
 * (n_tokens, dim), as `mx_silu_mul` (app/native/src/mx_fused_ops.c:36-42), written to out
 * (contiguous, may be NULL) and quantized to Q8_K into the workspace in the same pass (the down
 * projection's input). Rows of gate and of up are `ld` >= dim floats apart, so both may be the
 * halves of one gate|up output (ld = 2 * dim). Replaces `FusedOps.silu_mul`
 * (app/architectures/layers.py:53-57) plus that quantization. */
int mxa_silu_mul_q8_k(const float *gate, const float *up, long long ld, int n_tokens, int dim,
                      float *out, void *workspace, size_t workspace_bytes, void *stream);

/* Q8_K activation quantization of x (n_tokens, in_features) into the workspace layout
 * q int8 (n_tokens, K) | d fp32 (n_tokens, K/256) | bsums int16 (n_tokens, K/256, 16), each
 * part starting on a 256-byte boundary (see mxa_workspace_bytes).
 * Replaces `mx_quantize_row_q8_k` (app/native/src/mx_common.c:42-69). */
int mxa_quantize_q8_k(const float *x, int n_tokens, int in_features, void *workspace,
                      size_t workspace_bytes, void *stream);

/* Bit-exact dequantization of n_blocks packed blocks to fp32 (block_size values each).
 * Replaces `TorchDequantizer.dequantize` (app/gguf/dequant/torch_dequant.py:235-236), itself a
 * mirror of the numpy `QuantStrategy.dequantize`. */
int mxa_dequantize(int ggml_type, const void *blocks, long long n_blocks, float *out,
                   void *stream);

/* Rows `rows[0..n_rows)` (device int32 indices into the n_src_rows packed rows of `w`) of a
 * packed matrix with row_width values per row, dequantized bit-exactly to out (n_rows,
 * row_width) fp32; an index outside [0, n_src_rows) gives a row of NaN.
 * Replaces `mx_dequant_rows` (app/native/src/mx_dequant_rows.c:72-105) and the per-lookup
 * dequant of `DevicePackedEmbedding.forward` (app/architectures/device_packed.py:81-84). */
int mxa_dequant_rows(int ggml_type, const void *w, long long n_src_rows, const int32_t *rows,
                     int n_rows, int row_width, float *out, void *stream);

/* Reorders packed rows on the device: dst row i = src row order[i] for i < n_rows, rows of
 * row_bytes bytes (any GGUF type: a row is whole blocks); `order` is a device int32 array; an
 * index outside [0, n_src_rows) gives a row of zero bytes. src and dst must not overlap.
 * Replaces `PackedRows.reordered` (app/gguf/packed_rows.py:24-28), the host-side row permutation
 * the loader applies to packed attn_q / attn_k before `upload_packed`. */
int mxa_gather_rows(const void *src, long long n_src_rows, long long row_bytes,
                    const int32_t *order, int n_rows, void *dst, void *stream);

/* Measurement aid, with no counterpart in the reference: reads `bytes` bytes at `src` (device,
 * 16-byte aligned, a multiple of 16) once from HBM in one launch and computes nothing from them;
 * `sink` is a device word it may write. The time of this launch is the floor of any one-launch
 * kernel over the same bytes; bench.py reports the decode GEMV against it. */
int mxa_stream_read(const void *src, long long bytes, void *sink, void *stream);

/* Text of the last HIP error seen by this library on the calling thread ("" if none). */
const char *mxa_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* MATRICXON_AMD_H */
