// mxa_gemm for callers that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid it): the workspace the matmul needs beyond its inputs and
// outputs (the Q8_K activation blocks, or IQ4_XS prefill's bf16 split of x) lives in one
// file-scope device array instead of a caller buffer.
//
// Each device holds its own copy of `scratch` for the life of the process. Its device address is
// looked up once per device, with that device current, and kept; host code never passes the
// array's name itself (on the host it is only a stand-in symbol, not a device address). Calls on
// one device share the array, so calls that overlap on one device (several streams, or several
// host threads) race on it and must be ordered by the caller. Nothing in it has to start at zero:
// every byte a call reads was written earlier in the same call.
#include <atomic>
#include <mutex>

#include "../../include/matricxon_amd.h"
#include "mxa_kernels.hpp"

namespace {

constexpr size_t kScratchBytes = (size_t)16 << 20;  // MXA_STATIC_SCRATCH_BYTES
static_assert(kScratchBytes == MXA_STATIC_SCRATCH_BYTES, "header and source disagree");

__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];  // device address of `scratch`, per device
std::mutex g_lookup;

// This device's address of `scratch`, looked up on the first call on the device; nullptr (and the
// error text set) when the lookup fails.
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    mxa::set_last_error("mxa_gemm_static: no current HIP device");
    return nullptr;
  }
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  std::lock_guard<std::mutex> lock(g_lookup);
  p = g_scratch[dev].load(std::memory_order_relaxed);
  if (p == nullptr) {
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      mxa::set_last_error(hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace

extern "C" {

int mxa_gemm_static(int ggml_type, const void* w, const float* x, float* y, int n_tokens,
                    int out_features, int in_features, void* stream) {
  if (!mxa_supports(ggml_type, in_features) || n_tokens <= 0) return MXA_ERR_UNSUPPORTED;
  const size_t need = mxa_workspace_bytes(ggml_type, n_tokens, in_features);
  if (need > kScratchBytes) {
    mxa::set_last_error("mxa_gemm_static: the call needs more workspace than the static scratch "
                        "array holds (MXA_STATIC_SCRATCH_BYTES)");
    return MXA_ERR_WORKSPACE;
  }
  void* ws = scratch_on_current_device();
  if (ws == nullptr) return MXA_ERR_LAUNCH;
  return mxa_gemm(ggml_type, w, x, y, n_tokens, out_features, in_features, ws, kScratchBytes,
                  stream);
}

}  // extern "C"
