// head_rope.h -- the per-head q/k RMSNorm and half-layout RoPE of the decode
// step (runtime/model_runner_v2.py:155-163; rms_norm and apply_rope at
// runtime/model_runner.py:20-41), shared by the kernels that apply them so
// they produce the same bits.  One wave per head of D = 128: lane l owns
// elements l and l + 64, which are each other's RoPE partners.
#pragma once
#include "mx_device.h"

namespace hr {

// cos and sin of pos * inv_freq_l, inv_freq_l = 1 / theta^(2l / 128), fp32
// (runtime/model_runner.py:31-33).
__device__ __forceinline__ float2 rope_cs(float theta, int lane, int pos) {
    const float inv_freq = 1.0f / powf(theta, (float)(2 * lane) / 128.0f);
    const float ang = (float)pos * inv_freq;
    return make_float2(cosf(ang), sinf(ang));
}

// RMSNorm of the fp32 head (a = element lane, b = element lane + 64) with the
// bf16 weight (wa, wb), rounded to bf16, then RoPE in fp32 and bf16 again.
// Every lane of the wave must call it (the sum of squares is a wave sum, by
// DPP within rows of 16 lanes and then across the four rows).
__device__ __forceinline__ void norm_rope(float a, float b, float wa, float wb, float eps, float2 cs,
                                          uint16_t& ba, uint16_t& bb) {
    const float ss = mx::wave_reduce_dpp<false>(fmaf(a, a, b * b));
    const float r = 1.0f / sqrtf(ss / 128.0f + eps);
    const float na = mx::bf16_to_f32(mx::f32_to_bf16_rne((a * r) * wa));
    const float nb = mx::bf16_to_f32(mx::f32_to_bf16_rne((b * r) * wb));
    // out = x * cos + rotate_half(x) * sin
    const float ra = __fadd_rn(__fmul_rn(na, cs.x), __fmul_rn(-nb, cs.y));
    const float rb = __fadd_rn(__fmul_rn(nb, cs.x), __fmul_rn(na, cs.y));
    ba = mx::f32_to_bf16_rne(ra);
    bb = mx::f32_to_bf16_rne(rb);
}

}  // namespace hr
