// extern "C" entry points of libmatricxon_amd.so (declared in include/matricxon_amd.h):
// argument checks, workspace layout, kernel dispatch, status codes.
#include <stdio.h>
#include <string.h>

#include "../../include/matricxon_amd.h"
#include "mxa_kernels.hpp"

namespace {

thread_local char g_last_error[256] = "";

}  // namespace

namespace mxa {
void set_last_error(const char* text) { snprintf(g_last_error, sizeof g_last_error, "%s", text); }
}  // namespace mxa

namespace {

int check_launch() {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return MXA_OK;
  snprintf(g_last_error, sizeof g_last_error, "%s", hipGetErrorString(e));
  return MXA_ERR_LAUNCH;
}

bool known_type(int t) {
  return t == MXA_TYPE_Q8_0 || t == MXA_TYPE_Q4_K || t == MXA_TYPE_Q6_K || t == MXA_TYPE_IQ4_XS;
}

int block_elems(int t) { return t == MXA_TYPE_Q8_0 ? 32 : 256; }

int block_bytes(int t) {
  switch (t) {
    case MXA_TYPE_Q8_0: return 34;
    case MXA_TYPE_Q4_K: return 144;
    case MXA_TYPE_Q6_K: return 210;
    case MXA_TYPE_IQ4_XS: return 136;
    default: return 0;
  }
}

bool needs_q8k(int t) { return t != MXA_TYPE_IQ4_XS; }

// The kernels read packed blocks as dwords and activations / workspace as 16-byte vectors.
bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Up to fmax activation rows (the crossover, read once per call) the matmul kernel quantizes x
// itself (no workspace).
bool fused_quant(int n_tokens, int fmax) { return n_tokens <= fmax; }

mxa::Act make_act(const float* x, const mxa::ActBuffers* a, int k) {
  mxa::Act act;
  act.q = a ? a->q : nullptr;
  act.d = a ? a->d : nullptr;
  act.bsums = a ? a->bsums : nullptr;
  act.x = x;
  act.k = k;
  act.nb = k / mxa::QK;
  act.xsplit = nullptr;
  act.xbf16 = 0;
  return act;
}

// Workspace parts, each 256-byte aligned: the Q8_K activations (types other than IQ4_XS, more than
// fmax rows), then the bf16 split of x (IQ4_XS, kIq4MfmaMinRows rows or more).
size_t q8k_part(bool any_q8k, int n_tokens, int k, int fmax) {
  return any_q8k && !fused_quant(n_tokens, fmax) ? mxa::align256(mxa::act_bytes(n_tokens, k)) : 0;
}
size_t split_part(bool any_iq4, int n_tokens, int k) {
  return any_iq4 && n_tokens >= mxa::kIq4MfmaMinRows ? mxa::iq4_prefill_workspace(n_tokens, k) : 0;
}


// Workspace parts of a call on bfloat16 x, each 256-byte aligned: the Q8_K activations (any
// K-quant / Q8_0 weight: x is quantized into them whenever the floor-shaped decode kernel, which
// reads bfloat16 x itself, does not take the call), then x widened to float32 (any IQ4_XS weight,
// which multiplies float activations), then the IQ4_XS prefill split.
size_t widen_part(bool any_iq4, int n_tokens, int k) {
  return any_iq4 ? mxa::align256((size_t)n_tokens * k * 4) : 0;
}

int gemm_multi_core(int n, const int* types, const void* const* ws, const int* outs,
                    const void* x, bool xbf16, mxa::YOut y, int n_tokens, int in_features,
                    void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (n < 1 || n > 4 || types == nullptr || ws == nullptr || outs == nullptr)
    return MXA_ERR_UNSUPPORTED;
  if (x == nullptr || (y.v & ~(uintptr_t)1) == 0 || n_tokens <= 0 || !aligned(x, 16) ||
      !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  bool any_q8k = false, any_iq4 = false;
  long long total = 0;
  for (int i = 0; i < n; ++i) {
    if (!mxa_supports(types[i], in_features) || ws[i] == nullptr || outs[i] <= 0 ||
        !aligned(ws[i], 4))
      return MXA_ERR_UNSUPPORTED;
    any_q8k |= needs_q8k(types[i]);
    any_iq4 |= !needs_q8k(types[i]);
    total += outs[i];
  }
  const int fmax = mxa::fused_max_rows();
  const size_t q8k_bytes = xbf16 ? (any_q8k ? mxa::align256(mxa::act_bytes(n_tokens, in_features)) : 0)
                                 : q8k_part(any_q8k, n_tokens, in_features, fmax);
  const size_t widen_bytes = xbf16 ? widen_part(any_iq4, n_tokens, in_features) : 0;
  const size_t split_bytes = split_part(any_iq4, n_tokens, in_features);
  const size_t need = q8k_bytes + widen_bytes + split_bytes;
  mxa::DecodeSeg seg[4];
  long long c0 = 0;
  for (int i = 0; i < n; ++i) {
    seg[i] = mxa::DecodeSeg{types[i], (const uint8_t*)ws[i],
                            (long long)mxa_row_bytes(types[i], in_features), y.at(c0), outs[i]};
    c0 += outs[i];
  }
  if (xbf16 && !any_iq4 && n_tokens <= fmax) {
    // the floor-shaped decode kernel reads bfloat16 x and quantizes it itself (one launch, no
    // workspace); a launcher that declines has launched nothing
    mxa::Act a = make_act((const float*)x, nullptr, in_features);
    a.xbf16 = 1;
    const int st = n == 1 ? mxa::launch_gemv_wave_m(types[0], seg[0].w, seg[0].row_bytes, a, y,
                                                    total, n_tokens, outs[0], s)
                 : n_tokens == 1 ? mxa::launch_gemv_wave_multi(seg, n, a, s)
                                 : -1;
    if (st == 0) return check_launch();
  }
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return MXA_ERR_WORKSPACE;
  const float* xf = xbf16 ? nullptr : (const float*)x;
  if (widen_bytes > 0) {
    float* wide = (float*)((uint8_t*)workspace + q8k_bytes);
    mxa::launch_widen_bf16((const uint16_t*)x, wide, (long long)n_tokens * in_features, s);
    xf = wide;
  }
  mxa::ActBuffers buf{};
  const mxa::ActBuffers* abuf = nullptr;
  if (q8k_bytes > 0) {
    buf = mxa::act_layout(workspace, n_tokens, in_features);
    abuf = &buf;
    if (xbf16)
      mxa::launch_quantize_q8k_bf16((const uint16_t*)x, buf, n_tokens, in_features, s);
    else
      mxa::launch_quantize_q8k(xf, buf, n_tokens, in_features, s);
  }
  const int qst = check_launch();
  if (qst != MXA_OK) return qst;
  mxa::Act act = make_act(xf, abuf, in_features);
  if (split_bytes > 0) act.xsplit = (uint8_t*)workspace + q8k_bytes + widen_bytes;
  if (n > 1 && !any_iq4 && n_tokens <= 16) {  // decode: one launch for all weights
    int st = -1;
    if (n_tokens <= fmax) {
      st = mxa::launch_decode_multi(seg, n, act, total, n_tokens, s);
    } else {
      st = mxa::launch_bwave_multi(seg, n, act, total, n_tokens, s);
      if (st != 0) st = mxa::launch_bres_multi(seg, n, act, total, n_tokens, s);
      if (st != 0) st = mxa::launch_bstream_multi(seg, n, act, total, n_tokens, s);
    }
    if (st == 0) return check_launch();
  }
  for (int i = 0; i < n; ++i) {
    if (mxa::launch_matmul(types[i], seg[i].w, seg[i].row_bytes, act, seg[i].y, total, n_tokens,
                           outs[i], s) != 0)
      return MXA_ERR_UNSUPPORTED;
    const int st = check_launch();
    if (st != MXA_OK) return st;
  }
  return MXA_OK;
}

int gemm_q8k_core(int ggml_type, const void* w, const float* x, mxa::YOut y, int n_tokens,
                  int out_features, int in_features, const void* workspace,
                  size_t workspace_bytes, hipStream_t s) {
  if (!mxa_supports(ggml_type, in_features) || w == nullptr || n_tokens <= 0 ||
      out_features <= 0 || !aligned(w, 4) || !aligned(x, 16) || !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  mxa::ActBuffers buf{};
  const mxa::ActBuffers* abuf = nullptr;
  if (needs_q8k(ggml_type)) {
    if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, in_features))
      return MXA_ERR_WORKSPACE;
    buf = mxa::act_layout((void*)workspace, n_tokens, in_features);
    abuf = &buf;
  } else if (x == nullptr) {
    return MXA_ERR_UNSUPPORTED;
  }
  const mxa::Act act = make_act(x, abuf, in_features);
  const long long rb = (long long)mxa_row_bytes(ggml_type, in_features);
  if (mxa::launch_matmul(ggml_type, (const uint8_t*)w, rb, act, y, out_features, n_tokens,
                         out_features, s) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int gemm_multi_q8k_core(int n, const int* types, const void* const* ws, const int* outs,
                        mxa::YOut y, int n_tokens, int in_features, const void* workspace,
                        size_t workspace_bytes, hipStream_t s) {
  if (n < 1 || n > 4 || types == nullptr || ws == nullptr || outs == nullptr || n_tokens <= 0 ||
      !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  long long total = 0;
  for (int i = 0; i < n; ++i) {
    if (!mxa_supports(types[i], in_features) || !needs_q8k(types[i]) || ws[i] == nullptr ||
        outs[i] <= 0 || !aligned(ws[i], 4))
      return MXA_ERR_UNSUPPORTED;
    total += outs[i];
  }
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, in_features))
    return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers buf = mxa::act_layout((void*)workspace, n_tokens, in_features);
  const mxa::Act act = make_act(nullptr, &buf, in_features);
  mxa::DecodeSeg seg[4];
  long long c0 = 0;
  for (int i = 0; i < n; ++i) {
    seg[i] = mxa::DecodeSeg{types[i], (const uint8_t*)ws[i],
                            (long long)mxa_row_bytes(types[i], in_features), y.at(c0), outs[i]};
    c0 += outs[i];
  }
  if (n > 1 && n_tokens <= 16) {  // one launch for the group
    const int fmax = mxa::fused_max_rows();
    int st = n_tokens <= fmax ? mxa::launch_decode_multi(seg, n, act, total, n_tokens, s)
                              : mxa::launch_bwave_multi(seg, n, act, total, n_tokens, s);
    if (st != 0 && n_tokens > fmax) st = mxa::launch_bres_multi(seg, n, act, total, n_tokens, s);
    if (st != 0 && n_tokens > fmax)
      st = mxa::launch_bstream_multi(seg, n, act, total, n_tokens, s);
    if (st == 0) return check_launch();
  }
  for (int i = 0; i < n; ++i) {
    if (mxa::launch_matmul(types[i], seg[i].w, seg[i].row_bytes, act, seg[i].y, total, n_tokens,
                           outs[i], s) != 0)
      return MXA_ERR_UNSUPPORTED;
    const int st = check_launch();
    if (st != MXA_OK) return st;
  }
  return MXA_OK;
}

}  // namespace

extern "C" {

const char* mxa_build_info(void) {
  return "matricxon_amd gfx950: bit-exact dequant (Q8_0/Q4_K/Q6_K/IQ4_XS); decode M<=3: "
         "LDS-DMA wave GEMV with in-kernel Q8_K quantization; M 4..16: int8 MFMA gather kernel, "
         "each wave streaming its own block columns; prefill: int8 MFMA tiles (Q4_K/Q6_K/Q8_0), "
         "bf16 split MFMA (IQ4_XS)";
}

int mxa_supports(int ggml_type, int in_features) {
  return known_type(ggml_type) && in_features > 0 && in_features % mxa::QK == 0;
}

int mxa_supports_dequant_rows(int ggml_type, int row_width) {
  return mxa_supports(ggml_type, row_width);
}

void mxa_set_fused_max_tokens(int n_tokens) { mxa::set_fused_max_rows(n_tokens); }

int mxa_fused_max_tokens(void) { return mxa::fused_max_rows(); }

size_t mxa_row_bytes(int ggml_type, int in_features) {
  if (!mxa_supports(ggml_type, in_features)) return 0;
  return (size_t)(in_features / block_elems(ggml_type)) * block_bytes(ggml_type);
}

size_t mxa_workspace_bytes(int ggml_type, int n_tokens, int in_features) {
  if (!mxa_supports(ggml_type, in_features) || n_tokens <= 0) return 0;
  if (needs_q8k(ggml_type))
    return q8k_part(true, n_tokens, in_features, mxa::fused_max_rows());
  return split_part(true, n_tokens, in_features);
}

size_t mxa_workspace_bytes_bf16(int ggml_type, int n_tokens, int in_features) {
  if (!mxa_supports(ggml_type, in_features) || n_tokens <= 0) return 0;
  if (needs_q8k(ggml_type)) return mxa::align256(mxa::act_bytes(n_tokens, in_features));
  return widen_part(true, n_tokens, in_features) + split_part(true, n_tokens, in_features);
}

int mxa_quantize_q8_k_bf16(const void* x, int n_tokens, int in_features, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (x == nullptr || n_tokens <= 0 || in_features <= 0 || in_features % mxa::QK != 0 ||
      !aligned(x, 16) || !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, in_features))
    return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers a = mxa::act_layout(workspace, n_tokens, in_features);
  mxa::launch_quantize_q8k_bf16((const uint16_t*)x, a, n_tokens, in_features, (hipStream_t)stream);
  return check_launch();
}

int mxa_quantize_q8_k(const float* x, int n_tokens, int in_features, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (x == nullptr || n_tokens <= 0 || in_features <= 0 || in_features % mxa::QK != 0 ||
      !aligned(x, 16) || !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, in_features))
    return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers a = mxa::act_layout(workspace, n_tokens, in_features);
  mxa::launch_quantize_q8k(x, a, n_tokens, in_features, (hipStream_t)stream);
  return check_launch();
}

int mxa_gemm(int ggml_type, const void* w, const float* x, float* y, int n_tokens,
             int out_features, int in_features, void* workspace, size_t workspace_bytes,
             void* stream) {
  const int outs[1] = {out_features};
  const int types[1] = {ggml_type};
  const void* ws[1] = {w};
  return gemm_multi_core(1, types, ws, outs, x, false, mxa::YOut::f32(y), n_tokens, in_features,
                         workspace, workspace_bytes, (hipStream_t)stream);
}

int mxa_gemm_bf16(int ggml_type, const void* w, const void* x, void* y, int n_tokens,
                  int out_features, int in_features, void* workspace, size_t workspace_bytes,
                  void* stream) {
  if (!aligned(y, 2)) return MXA_ERR_UNSUPPORTED;
  const int outs[1] = {out_features};
  const int types[1] = {ggml_type};
  const void* ws[1] = {w};
  return gemm_multi_core(1, types, ws, outs, x, true, mxa::YOut::bf16(y), n_tokens, in_features,
                         workspace, workspace_bytes, (hipStream_t)stream);
}

int mxa_gemv_f32(int ggml_type, const void* w, const float* x, float* y, int n_tokens,
                 int out_features, int in_features, void* stream) {
  if (!mxa_supports(ggml_type, in_features) || w == nullptr || x == nullptr || y == nullptr ||
      n_tokens <= 0 || out_features <= 0 || !aligned(w, 4) || !aligned(x, 16))
    return MXA_ERR_UNSUPPORTED;
  const long long rb = (long long)mxa_row_bytes(ggml_type, in_features);
  const mxa::YOut yo = mxa::YOut::f32(y);
  for (int m0 = 0; m0 < n_tokens; m0 += 4) {  // activation rows m0 .. m0 + 3
    const int rows = n_tokens - m0 < 4 ? n_tokens - m0 : 4;
    if (mxa::launch_gemv_f32(ggml_type, (const uint8_t*)w, rb, x + (size_t)m0 * in_features,
                             in_features, yo.at((long long)m0 * out_features), out_features, rows,
                             out_features, (hipStream_t)stream) != 0)
      return MXA_ERR_UNSUPPORTED;
  }
  return check_launch();
}

int mxa_gemm_q8k(int ggml_type, const void* w, const float* x, float* y, int n_tokens,
                 int out_features, int in_features, const void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (y == nullptr) return MXA_ERR_UNSUPPORTED;
  return gemm_q8k_core(ggml_type, w, x, mxa::YOut::f32(y), n_tokens, out_features, in_features,
                       workspace, workspace_bytes, (hipStream_t)stream);
}

int mxa_gemm_q8k_bf16(int ggml_type, const void* w, void* y, int n_tokens, int out_features,
                      int in_features, const void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (y == nullptr || !aligned(y, 2) || !needs_q8k(ggml_type)) return MXA_ERR_UNSUPPORTED;
  return gemm_q8k_core(ggml_type, w, nullptr, mxa::YOut::bf16(y), n_tokens, out_features,
                       in_features, workspace, workspace_bytes, (hipStream_t)stream);
}

namespace {

int gemm_moe_core(int ggml_type, const void* w, long long expert_stride, int n_experts,
                  const float* x, const int32_t* offsets, int n_rows, int max_rows_per_expert,
                  mxa::YOut y, int out_features, int in_features, void* workspace,
                  size_t workspace_bytes, void* stream) {
  if (!mxa_supports(ggml_type, in_features) || w == nullptr || offsets == nullptr ||
      (y.v & ~(uintptr_t)1) == 0 || n_experts < 1 || n_rows < 1 || out_features < 1 ||
      max_rows_per_expert < 1 || !aligned(w, 4) || !aligned(x, 16) || !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  // every expert's weight starts as aligned as mxa_gemm asks of its w
  const long long rb = (long long)mxa_row_bytes(ggml_type, in_features);
  if (expert_stride < (long long)out_features * rb || expert_stride % 4 != 0)
    return MXA_ERR_UNSUPPORTED;
  if (!needs_q8k(ggml_type)) {  // IQ4_XS: float activations, no workspace
    if (x == nullptr) return MXA_ERR_UNSUPPORTED;
    const mxa::Act act = make_act(x, nullptr, in_features);
    if (mxa::launch_moe_lpb(ggml_type, (const uint8_t*)w, rb, expert_stride, n_experts, act,
                            offsets, n_rows, min(max_rows_per_expert, n_rows), y,
                            out_features, out_features, (hipStream_t)stream) != 0)
      return MXA_ERR_UNSUPPORTED;
    return check_launch();
  }
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_rows, in_features))
    return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers buf = mxa::act_layout(workspace, n_rows, in_features);
  const hipStream_t s = (hipStream_t)stream;
  if (x != nullptr) mxa::launch_quantize_q8k(x, buf, n_rows, in_features, s);
  const mxa::Act act = make_act(x, &buf, in_features);
  if (mxa::launch_moe_dec(ggml_type, (const uint8_t*)w, rb, expert_stride, n_experts, act,
                          offsets, n_rows, min(max_rows_per_expert, n_rows), y,
                          out_features, out_features, s) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

}  // namespace

int mxa_gemm_moe(int ggml_type, const void* w, long long expert_stride, int n_experts,
                 const float* x, const int32_t* offsets, int n_rows, int max_rows_per_expert,
                 float* y, int out_features, int in_features, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (y == nullptr) return MXA_ERR_UNSUPPORTED;
  return gemm_moe_core(ggml_type, w, expert_stride, n_experts, x, offsets, n_rows,
                       max_rows_per_expert, mxa::YOut::f32(y), out_features, in_features,
                       workspace, workspace_bytes, stream);
}

int mxa_gemm_moe_bf16(int ggml_type, const void* w, long long expert_stride, int n_experts,
                      const float* x, const int32_t* offsets, int n_rows, int max_rows_per_expert,
                      void* y, int out_features, int in_features, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (y == nullptr || !aligned(y, 2)) return MXA_ERR_UNSUPPORTED;
  return gemm_moe_core(ggml_type, w, expert_stride, n_experts, x, offsets, n_rows,
                       max_rows_per_expert, mxa::YOut::bf16(y), out_features, in_features,
                       workspace, workspace_bytes, stream);
}

int mxa_gemm_moe_pairs(int ggml_type, const void* w, long long expert_stride, int n_experts,
                       const int32_t* ids, int n_pairs, const float* x, int x_rows, float* y,
                       int out_features, int in_features, void* workspace, size_t workspace_bytes,
                       void* stream) {
  if (!mxa_supports(ggml_type, in_features) || !needs_q8k(ggml_type) || w == nullptr ||
      ids == nullptr || y == nullptr || n_experts < 1 || n_pairs < 1 || out_features < 1 ||
      (x_rows != 1 && x_rows != n_pairs) || !aligned(x, 16) || !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  const long long rb = (long long)mxa_row_bytes(ggml_type, in_features);
  if (expert_stride < (long long)out_features * rb) return MXA_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  const int x_step = x_rows == 1 ? 0 : 1;
  const mxa::YOut yo = mxa::YOut::f32(y);
  if (x != nullptr) {  // x quantized in the kernel where it can be
    const mxa::Act act = make_act(x, nullptr, in_features);
    if (mxa::launch_gemv_wave_pairs(ggml_type, (const uint8_t*)w, rb, expert_stride, ids,
                                    n_experts, n_pairs, x_step, act, yo, out_features, s) == 0)
      return check_launch();
  }
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(x_rows, in_features))
    return x == nullptr ? MXA_ERR_WORKSPACE : MXA_ERR_UNSUPPORTED;
  const mxa::ActBuffers buf = mxa::act_layout(workspace, x_rows, in_features);
  const mxa::Act act = make_act(nullptr, &buf, in_features);
  // x quantized into the workspace first (the workspace is the caller's scratch: on a shape the
  // kernel does not take, only it has been written)
  if (x != nullptr) mxa::launch_quantize_q8k(x, buf, x_rows, in_features, s);
  if (mxa::launch_gemv_wave_pairs(ggml_type, (const uint8_t*)w, rb, expert_stride, ids, n_experts,
                                  n_pairs, x_step, act, yo, out_features, s) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_gemm_moe_pairs_bf16(int ggml_type, const void* w, long long expert_stride, int n_experts,
                            const int32_t* ids, int n_pairs, const void* x, int x_rows, void* y,
                            int out_features, int in_features, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!mxa_supports(ggml_type, in_features) || !needs_q8k(ggml_type) || w == nullptr ||
      ids == nullptr || y == nullptr || n_experts < 1 || n_pairs < 1 || out_features < 1 ||
      (x_rows != 1 && x_rows != n_pairs) || !aligned(x, 16) || !aligned(y, 2) ||
      !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  const long long rb = (long long)mxa_row_bytes(ggml_type, in_features);
  if (expert_stride < (long long)out_features * rb) return MXA_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  const int x_step = x_rows == 1 ? 0 : 1;
  const mxa::YOut yo = mxa::YOut::bf16(y);
  if (x != nullptr) {  // bfloat16 x read and quantized in the kernel where it can be
    mxa::Act act = make_act((const float*)x, nullptr, in_features);
    act.xbf16 = 1;
    if (mxa::launch_gemv_wave_pairs(ggml_type, (const uint8_t*)w, rb, expert_stride, ids,
                                    n_experts, n_pairs, x_step, act, yo, out_features, s) == 0)
      return check_launch();
  }
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(x_rows, in_features))
    return x == nullptr ? MXA_ERR_WORKSPACE : MXA_ERR_UNSUPPORTED;
  const mxa::ActBuffers buf = mxa::act_layout(workspace, x_rows, in_features);
  const mxa::Act act = make_act(nullptr, &buf, in_features);
  if (x != nullptr) mxa::launch_quantize_q8k_bf16((const uint16_t*)x, buf, x_rows, in_features, s);
  if (mxa::launch_gemv_wave_pairs(ggml_type, (const uint8_t*)w, rb, expert_stride, ids, n_experts,
                                  n_pairs, x_step, act, yo, out_features, s) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_moe_route(const void* ids, int ids_int64, int n_tokens, int top_k, int n_experts,
                  int32_t* offsets, int32_t* pair_tok, int32_t* rows, int32_t* ids32,
                  void* stream) {
  if (mxa::launch_moe_route(ids, ids_int64 != 0, n_tokens, top_k, n_experts, offsets, pair_tok,
                            rows, ids32, (hipStream_t)stream) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_moe_combine(const float* down, const int32_t* rows, const int32_t* ids,
                    const float* weights, int n_tokens, int top_k, int n_embd, int round_bf16,
                    float* out, void* stream) {
  if (down == nullptr || ids == nullptr || weights == nullptr || out == nullptr)
    return MXA_ERR_UNSUPPORTED;
  if (mxa::launch_moe_combine(down, rows, ids, weights, n_tokens, top_k, n_embd, round_bf16 != 0,
                              out, (hipStream_t)stream) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_gemm_multi(int n, const int* types, const void* const* ws, const int* outs,
                   const float* x, float* y, int n_tokens, int in_features, void* workspace,
                   size_t workspace_bytes, void* stream) {
  return gemm_multi_core(n, types, ws, outs, x, false, mxa::YOut::f32(y), n_tokens, in_features,
                         workspace, workspace_bytes, (hipStream_t)stream);
}

int mxa_gemm_multi_bf16(int n, const int* types, const void* const* ws, const int* outs,
                        const void* x, void* y, int n_tokens, int in_features, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (!aligned(y, 2)) return MXA_ERR_UNSUPPORTED;
  return gemm_multi_core(n, types, ws, outs, x, true, mxa::YOut::bf16(y), n_tokens, in_features,
                         workspace, workspace_bytes, (hipStream_t)stream);
}

int mxa_gemm_multi_q8k(int n, const int* types, const void* const* ws, const int* outs, float* y,
                       int n_tokens, int in_features, const void* workspace,
                       size_t workspace_bytes, void* stream) {
  if (y == nullptr) return MXA_ERR_UNSUPPORTED;
  return gemm_multi_q8k_core(n, types, ws, outs, mxa::YOut::f32(y), n_tokens, in_features,
                             workspace, workspace_bytes, (hipStream_t)stream);
}

int mxa_gemm_multi_q8k_bf16(int n, const int* types, const void* const* ws, const int* outs,
                            void* y, int n_tokens, int in_features, const void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (y == nullptr || !aligned(y, 2)) return MXA_ERR_UNSUPPORTED;
  return gemm_multi_q8k_core(n, types, ws, outs, mxa::YOut::bf16(y), n_tokens, in_features,
                             workspace, workspace_bytes, (hipStream_t)stream);
}

int mxa_rms_norm_q8_k(const float* x, const float* weight, float eps, int n_tokens, int dim,
                      float* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (x == nullptr || weight == nullptr || n_tokens <= 0 || dim <= 0 || dim % mxa::QK != 0 ||
      !aligned(x, 16) || !aligned(weight, 4) || !aligned(out, 16) || !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, dim)) return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers a = mxa::act_layout(workspace, n_tokens, dim);
  mxa::launch_rms_norm_q8k(x, weight, eps, out, a, n_tokens, dim, (hipStream_t)stream);
  return check_launch();
}

int mxa_silu_mul_q8_k(const float* gate, const float* up, long long ld, int n_tokens, int dim,
                      float* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (gate == nullptr || up == nullptr || n_tokens <= 0 || dim <= 0 || dim % mxa::QK != 0 ||
      ld < dim || !aligned(gate, 4) || !aligned(up, 4) || !aligned(out, 16) ||
      !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, dim)) return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers a = mxa::act_layout(workspace, n_tokens, dim);
  mxa::launch_silu_mul_q8k(gate, up, ld, out, a, n_tokens, dim, (hipStream_t)stream);
  return check_launch();
}

int mxa_rms_norm_q8_k_bf16(const void* x, const void* weight, float eps, int n_tokens, int dim,
                           void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (x == nullptr || weight == nullptr || n_tokens <= 0 || dim <= 0 || dim % mxa::QK != 0 ||
      !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, dim)) return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers a = mxa::act_layout(workspace, n_tokens, dim);
  if (mxa::launch_rms_norm_q8k_bf16((const uint16_t*)x, (const uint16_t*)weight, eps,
                                    (uint16_t*)out, a, n_tokens, dim, (hipStream_t)stream) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_silu_mul_q8_k_bf16(const void* gate, const void* up, long long ld, int n_tokens, int dim,
                           void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (gate == nullptr || up == nullptr || n_tokens <= 0 || dim <= 0 || dim % mxa::QK != 0 ||
      ld < dim || !aligned(workspace, 16))
    return MXA_ERR_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < mxa::act_bytes(n_tokens, dim)) return MXA_ERR_WORKSPACE;
  const mxa::ActBuffers a = mxa::act_layout(workspace, n_tokens, dim);
  if (mxa::launch_silu_mul_q8k_bf16((const uint16_t*)gate, (const uint16_t*)up, ld, (uint16_t*)out,
                                    a, n_tokens, dim, (hipStream_t)stream) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_dequantize(int ggml_type, const void* blocks, long long n_blocks, float* out,
                   void* stream) {
  if (!known_type(ggml_type) || blocks == nullptr || out == nullptr || n_blocks <= 0)
    return MXA_ERR_UNSUPPORTED;
  if (mxa::launch_dequant(ggml_type, (const uint8_t*)blocks, nullptr, 0, 0, 1, n_blocks, out,
                          (hipStream_t)stream) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_dequant_rows(int ggml_type, const void* w, long long n_src_rows, const int32_t* rows,
                     int n_rows, int row_width, float* out, void* stream) {
  if (!mxa_supports(ggml_type, row_width) || w == nullptr || rows == nullptr || out == nullptr ||
      n_rows <= 0 || n_src_rows <= 0)
    return MXA_ERR_UNSUPPORTED;
  const int bpr = row_width / block_elems(ggml_type);
  const long long rb = (long long)mxa_row_bytes(ggml_type, row_width);
  if (mxa::launch_dequant(ggml_type, (const uint8_t*)w, rows, n_src_rows, rb, bpr,
                          (long long)n_rows * bpr, out, (hipStream_t)stream) != 0)
    return MXA_ERR_UNSUPPORTED;
  return check_launch();
}

int mxa_gather_rows(const void* src, long long n_src_rows, long long row_bytes,
                    const int32_t* order, int n_rows, void* dst, void* stream) {
  if (src == nullptr || order == nullptr || dst == nullptr || n_src_rows <= 0 || row_bytes <= 0 ||
      n_rows <= 0 || !aligned(order, 4))
    return MXA_ERR_UNSUPPORTED;
  mxa::launch_gather_rows(src, n_src_rows, row_bytes, order, n_rows, dst, (hipStream_t)stream);
  return check_launch();
}

int mxa_stream_read(const void* src, long long bytes, void* sink, void* stream) {
  if (src == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 != 0 || !aligned(src, 16) ||
      !aligned(sink, 4))
    return MXA_ERR_UNSUPPORTED;
  mxa::launch_stream_read(src, bytes, (uint32_t*)sink, (hipStream_t)stream);
  return check_launch();
}

const char* mxa_last_error(void) { return g_last_error; }

}  // extern "C"
