// Shader-clock probe for the benchmark: how fast the compute units actually
// run while another kernel (e.g. a large FP8 GEMM) keeps the GPU busy. Under
// a full matrix-core load the shader clock drops below its 2.4 GHz peak, and
// the dense FP8 peak (256 CUs x 8192 FLOP/clk) drops with it.
//
// One wave reads the shader-clock counter (s_memtime) and the constant-rate
// wall clock (s_memrealtime) at the start, spins on the wall clock for a
// fixed number of its ticks, and reads both again: cycles / seconds = sclk.
// The spin always ends (the wall clock advances whatever the shader clock).

#include "ifx_abi.h"

namespace {

__global__ __launch_bounds__(64) void sclk_probe_kernel(unsigned long long* out, unsigned long long ticks) {
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  unsigned long long r = r0;
  while (r - r0 < ticks) {
    __builtin_amdgcn_s_sleep(1);
    r = __builtin_amdgcn_s_memrealtime();
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = r - r0;
  }
}

}  // namespace

extern "C" {

int ifx_sclk_probe(void* out, int64_t wall_ticks, void* stream) {
  if (!out || wall_ticks <= 0 || wall_ticks > (int64_t(1) << 32)) return IFX_ERR_INVALID;
  if (!ifx::aligned16(out)) return IFX_ERR_ALIGN;
  hipLaunchKernelGGL(sclk_probe_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     static_cast<unsigned long long*>(out), static_cast<unsigned long long>(wall_ticks));
  return ifx::launch_status();
}

int ifx_wall_clock_khz(int* khz) {
  if (!khz) return IFX_ERR_INVALID;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev);
  return e == hipSuccess ? IFX_OK : static_cast<int>(e);
}

}  // extern "C"
