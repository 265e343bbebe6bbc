// kv_codec.h -- the reference's FP8 (E4M3) KV-cache byte codec
// (src/ext/mxfp4_decode.cu:355-364 e4m3_to_f32, :437-455 f32_to_e4m3), kept
// exactly because caches and attention outputs must match it: rounding half
// away from zero, |v| >= 248 saturating to 0x7F, subnormal codes read as
// m * 2^-6 (standard E4M3: m * 2^-9) and exponent-15 codes as 56 * (8 + m).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kv {

// The reference's E4M3 byte -> float.
__device__ __forceinline__ float e4m3_ref_decode(uint32_t b) {
    const uint32_t e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 0) v = (float)m * 0.015625f;                       // m * 2^-6
    else if (e == 15) v = (float)(8u + m) * 56.0f;              // 448 * (1 + m/8)
    else v = __uint_as_float(((e + 120u) << 23) | (m << 20));   // (1 + m/8) * 2^(e-7)
    return (b & 0x80u) ? -v : v;
}

// The reference's float -> E4M3 byte (round half away from zero).
__device__ __forceinline__ uint32_t e4m3_ref_encode(float v) {
    const uint32_t sign = v < 0.0f ? 0x80u : 0u;
    const float a = fabsf(v);
    if (a == 0.0f) return sign;
    int e;
    (void)frexpf(a, &e);                                 // a = f * 2^e, f in [0.5, 1)
    int eb = e + 6;
    const float man = a / ldexpf(1.0f, e - 1);           // [1, 2), exact
    int q = (int)lroundf((man - 1.0f) * 8.0f);
    if (q == 8) {
        q = 0;
        eb += 1;
    }
    if (eb <= 0) {
        int s = (int)lroundf(a * 64.0f);
        s = s > 7 ? 7 : (s < 0 ? 0 : s);
        return sign | (uint32_t)s;
    }
    if (eb >= 15) {
        eb = 15;
        q = 7;
    }
    return sign | ((uint32_t)(eb & 15) << 3) | (uint32_t)(q & 7);
}

// torch's float -> float8_e4m3fn, the cache write of the reference's batch
// step (runtime/model_runner_v2.py:256-257, k.to(torch.float8_e4m3fn)):
// round to nearest even; magnitudes that round past 448 (above 464),
// infinities and NaN give 0x7F, the format's NaN, with the input's sign;
// below 2^-6 the subnormal codes q * 2^-9.
__device__ __forceinline__ uint32_t e4m3_torch_encode(float v) {
    const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (!(a <= 464.0f)) return sign | 0x7Fu;
    if (a < 0.015625f) return sign | (uint32_t)(int)rintf(a * 512.0f);   // 0..8; 8 is the smallest normal
    const uint32_t bits = __float_as_uint(a);
    const float mant = __uint_as_float((bits & 0x7FFFFFu) | 0x3F800000u);   // [1, 2)
    int q = (int)rintf((mant - 1.0f) * 8.0f);                             // exact product, RNE
    uint32_t eb = (bits >> 23) - 120u;                                    // biased exponent e + 7
    if (q == 8) {
        q = 0;
        ++eb;
    }
    return sign | (eb << 3) | (uint32_t)q;
}

// Cache codecs of the KV write: the decode extension's kv_write (0) or
// torch's float8_e4m3fn conversion (1).
__device__ __forceinline__ uint32_t e4m3_encode(float v, int codec) {
    return codec ? e4m3_torch_encode(v) : e4m3_ref_encode(v);
}

}  // namespace kv
