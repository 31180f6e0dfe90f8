// Kernel choice for one packed weight (the role of mx_kernel_for / mx_gemm's dispatch,
// app/native/src/mx_gemm.c:25-108, 219-288):
//   K-quant / Q8_0, m_rows <= kDecodeMaxRows, IQ4_XS, m_rows <= 4
//                          pipelined lane-per-block decode kernel (mxa_gemv_lpb.hip)
//   Q8_0 / Q4_K / Q6_K     matrix-core kernels on the Q8_K workspace (mxa_mtile.hip dispatches:
//                          batched decode up to 16 rows, prefill tiles beyond)
//   IQ4_XS, >= 17 rows     bf16 matrix-core prefill on the split workspace (mxa_iq4.hip)
//   IQ4_XS, 5..16 rows     the decode kernel in passes of 4 rows (one summation order for decode)
#include "mxa_kernels.hpp"

namespace mxa {

int cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

int launch_matmul(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                  long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (m_rows <= (type == T_IQ4_XS ? kFusedQuantMaxRows : kDecodeMaxRows))
    return launch_gemv_lpb(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
  if (mtile_supported(type))
    return act.q != nullptr ? launch_mtile(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream) : -1;
  if (type != T_IQ4_XS) return -1;
  if (m_rows >= kIq4MfmaMinRows && act.xsplit != nullptr)
    return launch_iq4_prefill(w, row_bytes, act.x, act.xsplit, y, ldy, m_rows, act.k, n_rows, stream);
  for (int m0 = 0; m0 < m_rows; m0 += kFusedQuantMaxRows) {
    Act a = act;
    a.q = nullptr;
    a.x = act.x + (size_t)m0 * act.k;
    const int st = launch_gemv_lpb(type, w, row_bytes, a, y + (size_t)m0 * ldy, ldy,
                                   min(kFusedQuantMaxRows, m_rows - m0), n_rows, stream);
    if (st != 0) return st;
  }
  return 0;
}

}  // namespace mxa
