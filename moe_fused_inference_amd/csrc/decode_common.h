// decode_common.h -- activation splitting and word-exchange constants shared by the
// fused decode kernels (one layer per launch, and several layers per launch).
//
// There is no bf16 x FP4 MFMA, so a bf16 (or fp32) activation is split into
// kTerms E4M3 terms hi + mid + lo with E8M0 32-block scales s0 (the smallest
// power of two with amax <= 448 s0), s1 = s0 / 16 and s2 = s1 / 32: each term
// is the E4M3 rounding of what the terms before it left over.  Term 0 leaves
// at most 16 s0 (half its widest spacing, 32), i.e. <= 256 s1, which E4M3
// holds; term 1 then leaves at most 8 s1 = 256 s2, and term 2 at most
// 8 s2 = s0 / 64 <= 2^-13.8 of the block amax.  Only term 0's scale needs the
// block maximum (one cross-lane reduction per split).  The terms are rows 0..2
// of the A operand of v_mfma_scale_f32_16x16x128_f8f6f4.
#pragma once
#include "mx_device.h"

namespace dl {

constexpr int kSpinLimit = 1 << 22;   // polls per wait: about 1.3 s of polling (one round trip of ~0.3 us
                                      // each, s_sleep 1 between them) before the wait gives up
constexpr int kTerms = 3;             // E4M3 terms per activation value
constexpr int kMaxE = 8;
constexpr int kRecWords = 32;         // words per (slot, 32-block) record of h: one per value,
                                      // bytes 0..2 = its E4M3 terms, byte 3 of words 0..2 = the terms' codes
constexpr uint32_t kEmpty = 0xBADBAD7Fu;  // "no value yet": byte 0 is the E4M3 NaN code, which the term-0
                                          // byte of a finite value never is

// E8M0 code of the smallest 2^e with amax <= 448*2^e (E4M3 range), e in
// [-127, 127]; zero blocks get 127.
// Branch-free: both the normal and the subnormal exponent are computed and
// selected (amax is never negative).
__device__ __forceinline__ uint32_t e4m3_block_code(float amax) {
    const uint32_t bits = __float_as_uint(amax);
    const int ex = (int)(bits >> 23);
    const uint32_t frac = bits & 0x7FFFFFu;
    const int p = 31 - __clz((int)(frac | 1u));             // subnormal: leading bit of frac
    const uint32_t fn = (frac << (23 - p)) & 0x7FFFFFu;     // and frac normalised
    const int x = ex == 0 ? p - 149 : ex - 127;
    const uint32_t f = ex == 0 ? fn : frac;
    int e = (f <= 0x600000u) ? x - 8 : x - 7;               // (1+f) <= 1.75 -> 448 fits
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
    return amax > 0.0f ? (uint32_t)(e + 127) : 127u;        // zero (and NaN) blocks: 127
}

__device__ __forceinline__ float e8m0_value(uint32_t code) {
    return code > 0u ? __uint_as_float(code << 23) : __uint_as_float(0x00400000u);
}

// E8M0 codes of the three terms' scales from term 0's: s1 = s0 / 2^4, s2 = s0 / 2^9
// (clamped at the smallest code, which only makes a scale coarser, never overflowing).
constexpr int kTermShift[kTerms] = {0, 4, 9};
__device__ __forceinline__ uint32_t term_code(uint32_t code0, int t) {
    return code0 > (uint32_t)kTermShift[t] ? code0 - (uint32_t)kTermShift[t] : 0u;
}

// max over the 4 lanes of a quad (DPP quad permutes: no LDS round trip)
__device__ __forceinline__ float quad_max(float v) {
    const float a = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // xor 1
    v = fmaxf(v, a);
    const float b = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // xor 2
    return fmaxf(v, b);
}

// Splits 8 consecutive values of a 32-block (4 lanes per block, lane quad
// aligned) into kTerms E4M3 terms: word8[t] receives the 8 E4M3 bytes of term
// t and codes (byte t) the term's E8M0 scale code.  Each term is the E4M3
// rounding of what the previous terms left over, so the terms sum to the value
// up to the last term's rounding (at most 2^-13.8 of the block amax).
__device__ __forceinline__ void split8(float v[8], uint64_t word8[kTerms], uint32_t& codes) {
    codes = 0;
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, __builtin_fabsf(v[i]));
    const uint32_t code0 = e4m3_block_code(quad_max(am));
#pragma unroll
    for (int t = 0; t < kTerms; ++t) {
        const uint32_t code = term_code(code0, t);
        const float sc = e8m0_value(code);
        uint32_t word[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            mx::v2s p = {0, 0};
            p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, v[4 * h + 0], v[4 * h + 1], sc, false);
            p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, v[4 * h + 2], v[4 * h + 3], sc, true);
            word[h] = ((uint32_t)(uint16_t)p[0]) | ((uint32_t)(uint16_t)p[1] << 16);
            typedef float v2f __attribute__((ext_vector_type(2)));
            const v2f d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word[h], sc, false);
            const v2f d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word[h], sc, true);
            v[4 * h + 0] -= d0[0];
            v[4 * h + 1] -= d0[1];
            v[4 * h + 2] -= d1[0];
            v[4 * h + 3] -= d1[1];
        }
        word8[t] = (uint64_t)word[0] | ((uint64_t)word[1] << 32);
        codes |= code << (8 * t);
    }
}

// max over the 8 lanes of a half row: the quad maximum, then the other quad's
// through the half-row mirror (DPP)
__device__ __forceinline__ float oct_max(float v) {
    v = quad_max(v);
    return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));
}

// Splits 4 consecutive values of a 32-block (8 lanes per block, aligned to 8
// lanes) into kTerms E4M3 terms, with split8's arithmetic: word4[t] receives
// the 4 E4M3 bytes of term t and codes (byte t) the term's E8M0 scale code.
__device__ __forceinline__ void split4(float v[4], uint32_t word4[kTerms], uint32_t& codes) {
    codes = 0;
    const float am = fmaxf(fmaxf(__builtin_fabsf(v[0]), __builtin_fabsf(v[1])),
                           fmaxf(__builtin_fabsf(v[2]), __builtin_fabsf(v[3])));
    const uint32_t code0 = e4m3_block_code(oct_max(am));
#pragma unroll
    for (int t = 0; t < kTerms; ++t) {
        const uint32_t code = term_code(code0, t);
        const float sc = e8m0_value(code);
        mx::v2s p = {0, 0};
        p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, v[0], v[1], sc, false);
        p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, v[2], v[3], sc, true);
        const uint32_t word = ((uint32_t)(uint16_t)p[0]) | ((uint32_t)(uint16_t)p[1] << 16);
        typedef float v2f __attribute__((ext_vector_type(2)));
        const v2f d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, sc, false);
        const v2f d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, sc, true);
        v[0] -= d0[0];
        v[1] -= d0[1];
        v[2] -= d1[0];
        v[3] -= d1[1];
        word4[t] = word;
        codes |= code << (8 * t);
    }
}

// max over lanes 0..15 and over 16..31 (each row of 16 lanes), then of both
// rows, for a value held by lanes 0..31: DPP within rows, readlane across.
__device__ __forceinline__ float max32(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));   // quad xor 1
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));   // quad xor 2
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));  // row half-mirror
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));  // row mirror
    return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)));
}

// Splits a 32-block held one value per lane (lanes 0..31) into kTerms E4M3
// terms, as split8 does: returns the lane's term bytes (byte t = term t) and
// the block's codes (byte t = E8M0 code of term t, the same in every lane).
__device__ __forceinline__ uint32_t split32(float v, uint32_t& codes) {
    uint32_t bytes = 0;
    codes = 0;
    const uint32_t code0 = e4m3_block_code(max32(__builtin_fabsf(v)));
#pragma unroll
    for (int t = 0; t < kTerms; ++t) {
        const uint32_t code = term_code(code0, t);
        const float sc = e8m0_value(code);
        mx::v2s p = {0, 0};
        p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, v, 0.0f, sc, false);
        const uint32_t b = (uint32_t)(uint16_t)p[0] & 0xFFu;
        typedef float v2f __attribute__((ext_vector_type(2)));
        const v2f d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(b, sc, false);
        v -= d[0];
        bytes |= b << (8 * t);
        codes |= code << (8 * t);
    }
    return bytes;
}

// Unconditional load from an always-valid (clamped) address, value selected
// afterwards: keeps every load of a phase in one basic block so the compiler
// can wait for exactly the loads a computation needs.
template <typename T>
__device__ __forceinline__ T ld_sel(const T* p, bool ok, T zero) {
    const T v = *p;
    return ok ? v : zero;
}

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ mx::v8i cat8(uint4 lo, uint4 hi) {
    mx::v8i a = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    return a;
}

}  // namespace dl
