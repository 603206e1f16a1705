// Measurement probe (no counterpart in the reference):
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
