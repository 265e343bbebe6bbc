// quant_rows.h -- one thread's share of the activation -> MXFP4 quantizer
// (quant.hip): eight consecutive elements of a row, four consecutive lanes per
// 32-block.  Shared by quantize_rows_kernel and the kernels that run the
// quantization beside other work in one launch, so both give the same bits.
#pragma once
#include "mx_device.h"
#include "mxfp4_hip.h"

namespace mxq {

template <int SRC>
__device__ __forceinline__ float load_elem(const void* x, int64_t idx) {
    if (SRC == MXFP4_DT_BF16) return mx::bf16_to_f32(static_cast<const uint16_t*>(x)[idx]);
    if (SRC == MXFP4_DT_F16) return mx::f16_to_f32(static_cast<const uint16_t*>(x)[idx]);
    return static_cast<const float*>(x)[idx];
}

// Loads 8 consecutive elements starting at row offset k0 (16-byte aligned
// vector path when `vec` holds, element path with zero fill otherwise).
template <int SRC>
__device__ __forceinline__ void load8(const void* x, int64_t base, int k0, int K, bool vec,
                                      float v[8]) {
    if (vec && k0 + 8 <= K) {
        if (SRC == MXFP4_DT_F32) {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base + k0);
            float4 a = p[0], b = p[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base + k0);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint16_t lo = (uint16_t)(w[i] & 0xFFFFu), hi = (uint16_t)(w[i] >> 16);
                if (SRC == MXFP4_DT_BF16) {
                    v[2 * i] = mx::bf16_to_f32(lo);
                    v[2 * i + 1] = mx::bf16_to_f32(hi);
                } else {
                    v[2 * i] = mx::f16_to_f32(lo);
                    v[2 * i + 1] = mx::f16_to_f32(hi);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? load_elem<SRC>(x, base + k0 + i) : 0.0f;
    }
}

// RND: 0 none, 1 round each element to fp16 first, 2 to bf16 first.
// Unit u (elements 8u .. 8u+7) of row `row`; rows >= M and units past the
// row's Kp/8 write nothing.  Needs the four lanes of a 32-block in one quad.
template <int SRC, int RND>
__device__ __forceinline__ void quantize_unit(const void* __restrict__ x, int64_t ldx, int M, int K, int Kp,
                                              bool vecok, int64_t row, int u, uint8_t* __restrict__ q,
                                              uint8_t* __restrict__ s) {
    const int upr = Kp >> 3;  // 8-element units per row
    const int vec = vecok ? 1 : 0;
    const bool valid = row < M && u < upr;
    const int k0 = u * 8;
    float v[8];
    if (valid) {
        load8<SRC>(x, row * ldx, k0, K, vec != 0, v);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    if (RND == 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = mx::round_to_f16(v[i]);
    }
    if (RND == 2) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(v[i]));
    }
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, __builtin_fabsf(v[i]));
    // the block's four lanes: quad max by DPP
    am = fmaxf(am, mx::dpp<mx::kDppQuadXor1>(am));
    am = fmaxf(am, mx::dpp<mx::kDppQuadXor2>(am));
    const uint32_t code = mx::e8m0_code(am);
    // fp32 input without rounding keeps the software codes (up to 24 significant bits)
    const uint32_t packed = (SRC == MXFP4_DT_F32 && RND == 0) ? mx::e2m1_pack8(v, mx::e8m0_inv_scale(code))
                                                              : mx::e2m1_pack8_short(v, mx::e8m0_inv_scale(code));
    if (valid) {
        *reinterpret_cast<uint32_t*>(q + row * (int64_t)(Kp >> 1) + (u << 2)) = packed;
        if ((u & 3) == 0) s[row * (int64_t)(Kp >> 5) + (u >> 2)] = (uint8_t)code;
    }
}

}  // namespace mxq
