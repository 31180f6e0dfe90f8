// Kernel choice for one packed weight (the role of mx_kernel_for / mx_gemm's dispatch,
// app/native/src/mx_gemm.c:25-112, 123-194):
//   K-quant / Q8_0, m_rows <= kDecodeMaxRows, IQ4_XS, m_rows <= 4
//                          pipelined lane-per-block decode kernel (mxa_gemv_lpb.hip)
//   Q8_0 / Q4_K / Q6_K     matrix-core kernels on the Q8_K workspace (mxa_mtile.hip dispatches:
//                          batched decode up to 16 rows, prefill tiles beyond)
//   IQ4_XS, >= 17 rows     bf16 matrix-core prefill on the split workspace (mxa_iq4.hip)
//   IQ4_XS, 5..16 rows     the decode kernel in passes of 4 rows (one summation order for decode)
#include <atomic>
#include <mutex>
#include <set>
#include <tuple>

#include "mxa_kernels.hpp"

namespace mxa {

namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];  // 0 until first asked for on that device
std::atomic<int> g_fused_max_rows{kDecodeMaxRows};

int current_device() {
  int dev = 0;
  return hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices ? dev : 0;
}
}  // namespace

int cu_count() {
  const int dev = current_device();
  int n = g_cu_count[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int v = 0;
    n = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
            ? v
            : 256;
    g_cu_count[dev].store(n, std::memory_order_relaxed);  // every thread computes the same value
  }
  return n;
}

void allow_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::tuple<const void*, int, int>> done;  // (kernel, device, bytes)
  const int dev = current_device();
  std::lock_guard<std::mutex> lock(mu);
  if (done.emplace(kernel, dev, bytes).second)
    (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

int fused_max_rows() { return g_fused_max_rows.load(std::memory_order_relaxed); }

void set_fused_max_rows(int n) {
  g_fused_max_rows.store(n < 0 ? 0 : n > kFusedQuantMaxRows ? kFusedQuantMaxRows : n,
                         std::memory_order_relaxed);
}

int launch_matmul(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                  long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (type == T_IQ4_XS || act.q == nullptr) {
    // IQ4_XS up to kFusedQuantMaxRows rows; K-quants whose x the caller left unquantized (the
    // decode kernel quantizes it)
    if (m_rows <= kFusedQuantMaxRows)
      return launch_gemv_lpb(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    if (type != T_IQ4_XS) return -1;
  } else if (m_rows <= fused_max_rows()) {
    // Q8_K already in the workspace: either kernel gives the same bits; the crossover picks
    return launch_gemv_lpb(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
  }
  if (mtile_supported(type))
    return launch_mtile(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
  if (type != T_IQ4_XS) return -1;
  if (m_rows >= kIq4MfmaMinRows && act.xsplit != nullptr)
    return launch_iq4_prefill(w, row_bytes, act.x, act.xsplit, y, ldy, m_rows, act.k, n_rows, stream);
  for (int m0 = 0; m0 < m_rows; m0 += kFusedQuantMaxRows) {
    Act a = act;
    a.q = nullptr;
    a.x = act.x + (size_t)m0 * act.k;
    const int st = launch_gemv_lpb(type, w, row_bytes, a, y.at((size_t)m0 * ldy), ldy,
                                   min(kFusedQuantMaxRows, m_rows - m0), n_rows, stream);
    if (st != 0) return st;
  }
  return 0;
}

}  // namespace mxa
