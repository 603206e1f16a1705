// icpp_gemm_noalloc: icpp_gemm for callers that cannot allocate device memory.
//
// icpp_gemm's split-K path keeps fp32 partials [splits][M][N] in a caller
// workspace.  This entry point keeps them in `scratch`, a file-scope device array
// of ICPP_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds from
// module load until the process ends.  Its device address is resolved once per
// device with hipGetSymbolAddress (on the host, the array's name is only a stand-in
// for the symbol, never a device address) and cached; afterwards a call performs
// no allocation: argument checks, then the same kernels as icpp_gemm.
//
// Nothing in the scratch has to start at zero: the GEMM kernel writes every
// partial element (m < M, n < N) of every K slice before the reduce kernel, which
// is stream-ordered after it, reads them.  All calls on one GPU share the array,
// so calls that overlap in time on one GPU (different streams, or host threads
// racing to enqueue on different streams) race on it; calls serialised on one
// stream are safe.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/icpp_hip.h"

namespace icpp {
int set_last_error(int code, const char* msg);  // icpp_abi.hip
}

static __device__ __align__(256) unsigned char scratch[ICPP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mutex;

// The current device's address of `scratch`, resolved on the first call on that device.
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return icpp::set_last_error((int)e, "icpp_gemm_noalloc: hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return icpp::set_last_error(ICPP_E_ARG, "icpp_gemm_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return icpp::set_last_error(e != hipSuccess ? (int)e : ICPP_E_ARG,
                                  "icpp_gemm_noalloc: hipGetSymbolAddress(scratch) failed");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ICPP_OK;
}

}  // namespace

extern "C" int icpp_gemm_noalloc(int inst, const void* A, const void* B, const void* bias, void* C,
                                 int M, int N, int K, int lda, int ldb, int ldc, int act,
                                 float scale_a, float scale_b, int split_k, void* stream) {
  if (split_k > 1) {
    if (M <= 0 || N <= 0) return icpp::set_last_error(ICPP_E_SHAPE, "icpp_gemm_noalloc: empty shape");
    const uint64_t need = (uint64_t)split_k * (uint64_t)M * (uint64_t)N * sizeof(float);
    if (need > ICPP_NOALLOC_SCRATCH_BYTES)
      return icpp::set_last_error(ICPP_E_WORKSPACE,
                                  "icpp_gemm_noalloc: split-K partials (split_k * M * N * 4 bytes) exceed the "
                                  "static scratch of ICPP_NOALLOC_SCRATCH_BYTES; use icpp_gemm with a workspace");
    void* ws = nullptr;
    const int rc = scratch_for_current_device(&ws);
    if (rc != ICPP_OK) return rc;
    return icpp_gemm(inst, A, B, bias, C, M, N, K, lda, ldb, ldc, act, scale_a, scale_b, split_k, ws,
                     (size_t)ICPP_NOALLOC_SCRATCH_BYTES, stream);
  }
  return icpp_gemm(inst, A, B, bias, C, M, N, K, lda, ldb, ldc, act, scale_a, scale_b, split_k, nullptr, 0, stream);
}
