// selftest.hip -- device-side checks of shared reduction helpers, exported
// for the GPU tests (no counterpart in the reference).
//
// mxfp4_selftest_wave_sum: for every wave of 64 input values, the wave sum
// as the RMSNorm kernels compute it (mx::wave_sum_butterfly: permlane swaps
// and DPP) and as the plain xor butterfly of __shfl_xor, each lane's result
// in both outputs, so a test can require the two to agree bit for bit on
// every lane (including inf / NaN propagation).
#include "mx_device.h"
#include "mx_host.h"

namespace {
__global__ __launch_bounds__(64) void wave_sum_kernel(const float* __restrict__ in, float* __restrict__ out_dpp,
                                                      float* __restrict__ out_xor) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const float v = in[i];
    float s = v;
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
    out_xor[i] = s;
    out_dpp[i] = mx::wave_sum_butterfly(v);
}
}  // namespace

extern "C" int mxfp4_selftest_wave_sum(const float* in, float* out_butterfly, float* out_xor, int n_waves,
                                       void* stream) {
    MXH_REQUIRE(in && out_butterfly && out_xor, "selftest_wave_sum: null pointer");
    MXH_REQUIRE(n_waves > 0 && n_waves <= (1 << 20), "selftest_wave_sum: n_waves=%d", n_waves);
    hipLaunchKernelGGL(wave_sum_kernel, dim3((unsigned)n_waves), dim3(64), 0, mxh::as_stream(stream), in,
                       out_butterfly, out_xor);
    return mxh::launch_status("selftest_wave_sum");
}
