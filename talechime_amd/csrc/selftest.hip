// selftest.hip -- on-device checks of the approximations the kernels build
// their error bounds on, where the instruction they use exists only on the
// GPU (and so cannot be checked by the host-side table generator).
//
//   tc_selftest_exp_approx: the largest distance, in ulps, between
//   exp_approx(d) and tc_expf_cr(d) over every float d in [-87, 0].  The
//   exact sequential sum takes approximate terms to be within kSeqErr = 2^-21
//   relative of glibc's expf; glibc is within 1 ulp of tc_expf_cr, so a
//   distance of at most 3 ulps (4 ulps <= 2^-21 relative) keeps that bound.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tc_device.h"

namespace {

__device__ unsigned int g_max_ulps;

__global__ void __launch_bounds__(256) k_exp_approx(uint32_t lo, uint32_t hi) {
  // negative floats: bits lo (= -0) .. hi (= -87), magnitudes increasing with the bits
  const uint32_t stride = gridDim.x * blockDim.x;
  unsigned int worst = 0;
  for (uint32_t b = lo + blockIdx.x * blockDim.x + threadIdx.x; b <= hi && b >= lo; b += stride) {
    const float d = __uint_as_float(b);
    const float ap = tc::exp_approx(d);
    const float cr = (float)tc_exp_d((double)d);
    const uint32_t ua = __float_as_uint(ap), uc = __float_as_uint(cr);
    const unsigned int diff = (!(ap >= 0.0f) || ap == __builtin_inff()) ? 0xffffffffu : (ua > uc ? ua - uc : uc - ua);
    worst = diff > worst ? diff : worst;
    if (b > hi - stride) break;  // the next step would pass hi (or wrap)
  }
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned int v = __shfl_xor(worst, o);
    worst = v > worst ? v : worst;
  }
  if ((threadIdx.x & 63) == 0) atomicMax(&g_max_ulps, worst);
}

}  // namespace

extern "C" int tc_selftest_exp_approx(unsigned int* max_ulps) {
  const unsigned int zero = 0;
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_max_ulps), &zero, sizeof(zero)) != hipSuccess) return -1;
  const uint32_t lo = 0x80000000u, hi = 0xc2ae0000u;  // -0 .. -87
  hipLaunchKernelGGL(k_exp_approx, dim3(16384), dim3(256), 0, 0, lo, hi);
  if (hipGetLastError() != hipSuccess) return -2;
  if (hipDeviceSynchronize() != hipSuccess) return -3;
  if (hipMemcpyFromSymbol(max_ulps, HIP_SYMBOL(g_max_ulps), sizeof(unsigned int)) != hipSuccess) return -4;
  return 0;
}
