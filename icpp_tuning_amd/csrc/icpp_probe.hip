// Measurement probes (no counterpart in the reference):
//
// Shader-clock probe: the average shader clock over a stretch of wall time.
//
// One wave reads the shader-clock counter (s_memtime, one tick per shader clock
// cycle) and the constant 100 MHz real-time counter (s_memrealtime) at the start,
// sleeps until `ticks` real-time ticks have passed, and reads both again.  Run on
// its own stream beside a kernel under test, it reports the clock the chip
// sustained under that load (the figure that turns a datasheet peak, quoted at the
// 2.4 GHz maximum, into the peak reachable at the clock actually held).
//
// The wait is bounded by the real-time counter alone, so the wave always exits;
// the launcher caps `ticks` at 10 s.  s_sleep keeps the wave off the issue port.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/icpp_hip.h"

namespace icpp {
int set_last_error(int code, const char* msg);  // icpp_abi.hip
}

namespace {

__global__ void __launch_bounds__(64) clock_probe_kernel(unsigned long long* out, unsigned long long ticks) {
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  unsigned long long r = r0;
  while (r - r0 < ticks) {
    __builtin_amdgcn_s_sleep(32);
    r = __builtin_amdgcn_s_memrealtime();
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = r - r0;
  }
}

}  // namespace

// Read-bandwidth probe: `wgs` workgroups of `threads` threads read a rows x ld-byte
// matrix region, workgroup w a stripe of `stripe` bytes x `rows_per_wg` rows
// (column block w % (ld / stripe), row block w / (ld / stripe)), 16 bytes per lane
// and load, 8 loads in flight per lane.  A lane keeps one 16-byte column of the
// stripe and walks down its rows (threads / (stripe / 16) rows per load), so the
// address arithmetic is one add per load and the probe measures the memory path,
// not the ALU.  Consecutive workgroups of one XCD take neighbouring stripes.  With
// `passes` > 1 a workgroup reads its stripe that many times (later passes hit L2);
// with `shared` every workgroup reads stripe 0 (the same lines).  The loaded data is
// folded into a value written only if it equals a sentinel, so no load is dropped.
__global__ void __launch_bounds__(1024) read_probe_kernel(const char* __restrict__ base, unsigned ld, int stripe,
                                                          int rows_per_wg, int passes, int shared, int* sink) {
  int slot = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) slot = (slot & 7) * (nb >> 3) + (slot >> 3);
  if (shared) slot = 0;
  const int cpr = stripe / 16;                      // 16-byte chunks per row; divides blockDim.x
  const int ncb = (int)(ld / (unsigned)stripe);
  const int cb = slot % ncb, rb = slot / ncb;
  const int step = (int)blockDim.x / cpr;           // rows one load of the workgroup covers
  const char* p0 = base + (size_t)rb * rows_per_wg * ld + (size_t)cb * stripe + (threadIdx.x % cpr) * 16;
  const int r0 = (int)threadIdx.x / cpr;
  const size_t dstep = (size_t)step * ld;
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 acc = {0, 0, 0, 0};
  for (int pass = 0; pass < passes; ++pass) {
    const char* p = p0 + (size_t)r0 * ld;
    for (int r = r0; r < rows_per_wg; r += 8 * step) {
      i32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = (r + u * step < rows_per_wg) ? *(const i32x4*)(p + u * dstep) : i32x4{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < 8; ++u) acc ^= v[u];
      p += 8 * dstep;
    }
  }
  const int x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x5eed1e55) sink[blockIdx.x] = x;
}

extern "C" int icpp_read_probe(const void* base, size_t bytes, unsigned ld, int stripe, int rows_per_wg, int threads,
                               int passes, int shared, int* sink, size_t sink_ints, void* stream) {
  if (!base || !sink) return icpp::set_last_error(ICPP_E_ARG, "icpp_read_probe: null pointer");
  if (ld == 0 || stripe < 16 || stripe % 16 || ld % (unsigned)stripe || rows_per_wg <= 0 ||
      (threads != 256 && threads != 512 && threads != 1024) || threads % (stripe / 16) || passes < 1 || passes > 64)
    return icpp::set_last_error(ICPP_E_ARG, "icpp_read_probe: need 16 | stripe | ld, stripe / 16 | threads, rows > 0, "
                                            "threads 256/512/1024, passes 1-64");
  const size_t rows = bytes / ld;
  if (rows == 0 || rows % (size_t)rows_per_wg)
    return icpp::set_last_error(ICPP_E_SHAPE, "icpp_read_probe: bytes / ld must be a multiple of rows_per_wg");
  const size_t wgs = (ld / stripe) * (rows / rows_per_wg);
  if (wgs > sink_ints || wgs > 0x7FFFFFFF)
    return icpp::set_last_error(ICPP_E_SHAPE, "icpp_read_probe: more workgroups than sink entries");
  if ((reinterpret_cast<uintptr_t>(base) & 15) != 0)
    return icpp::set_last_error(ICPP_E_ARG, "icpp_read_probe: base must be 16-byte aligned");
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)wgs), dim3(threads), 0, (hipStream_t)stream, (const char*)base,
                     ld, stripe, rows_per_wg, passes, shared ? 1 : 0, sink);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return icpp::set_last_error((int)e, "icpp_read_probe: launch failed");
  return ICPP_OK;
}

extern "C" int icpp_clock_probe(unsigned long long* out, double seconds, void* stream) {
  if (!out) return icpp::set_last_error(ICPP_E_ARG, "icpp_clock_probe: null output");
  if (!(seconds > 0.0) || seconds > 10.0)
    return icpp::set_last_error(ICPP_E_ARG, "icpp_clock_probe: seconds must be in (0, 10]");
  if ((reinterpret_cast<uintptr_t>(out) & 7) != 0)
    return icpp::set_last_error(ICPP_E_ARG, "icpp_clock_probe: output must be 8-byte aligned");
  const unsigned long long ticks = (unsigned long long)(seconds * 1e8);  // 100 MHz real-time counter
  hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, out, ticks);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return icpp::set_last_error((int)e, "icpp_clock_probe: launch failed");
  return ICPP_OK;
}
