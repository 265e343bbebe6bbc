// quant.hip -- bit-exact activation -> MXFP4 quantizer for gfx950.
//
// Contract: quant/fp4_format.py (E2M1 ties-up, smallest power-of-two E8M0
// scale, LSB-first nibbles), applied per 32-block of each row exactly as
// quant/quantize_mxfp4.py:124-147 does for weights and as the reference's
// prequant kernel does for activations (src/ext/mxfp4_decode.cu:24-50).
//
// Layout of the work: four consecutive lanes own one 32-block, eight
// consecutive elements each.  A wave therefore reads 64 x 16 contiguous bytes
// of bf16 input (fully coalesced), reduces the block amax with two DPP quad
// exchanges, and each lane writes the 4 bytes holding
// its 8 nibbles -- again contiguous across the wave.  The lane with quad index
// 0 writes the block's scale byte.  HBM-bound: 2 B read + 0.53 B written per
// element for bf16 input.
#include "mx_device.h"
#include "mx_host.h"

namespace {

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
// Workgroup (row group blockIdx.x, unit segment blockIdx.y): 2^lt threads per
// row (the units of a row rounded up to a power of two, at most 256), so the
// row and unit of a thread are shifts and masks, not a division.
template <int SRC, int RND>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const void* __restrict__ x, int64_t ldx,
                                                            int M, int K, int Kp, int vec, int lt,
                                                            uint8_t* __restrict__ q,
                                                            uint8_t* __restrict__ s) {
    const int upr = Kp >> 3;  // 8-element units per row
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * (256 >> lt) + (tid >> lt);
    const int u = (int)blockIdx.y * (1 << lt) + (tid & ((1 << lt) - 1));
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

template <int SRC, int RND>
void launch_quant(const void* x, int64_t ldx, int M, int K, int Kp, int vec, uint8_t* q, uint8_t* s,
                  hipStream_t st) {
    const int upr = Kp >> 3;
    int lt = 2;                                    // Kp >= 32: at least 4 units per row
    while ((1 << lt) < upr && lt < 8) ++lt;
    const int rpw = 256 >> lt;
    const unsigned gx = (unsigned)((M + rpw - 1) / rpw), gy = (unsigned)((upr + (1 << lt) - 1) >> lt);
    hipLaunchKernelGGL((quantize_rows_kernel<SRC, RND>), dim3(gx, gy), dim3(256), 0, st,
                       x, ldx, M, K, Kp, vec, lt, q, s);
}

}  // namespace

namespace mxh {
// Shared by mxfp4_linear_forward.
int quantize_rows_impl(const void* x, int src_dtype, int round_to_f16, int64_t ldx, int M, int K,
                       int Kp, uint8_t* q, uint8_t* s, hipStream_t st) {
    MXH_REQUIRE(x && q && s, "quantize: null pointer");
    MXH_REQUIRE(M >= 0 && K >= 0, "quantize: negative size (M=%d K=%d)", M, K);
    MXH_REQUIRE(Kp % 32 == 0 && Kp >= K, "quantize: Kp=%d must be a multiple of 32 and >= K=%d", Kp, K);
    MXH_REQUIRE(ldx >= K, "quantize: row stride %lld < K=%d", (long long)ldx, K);
    MXH_REQUIRE(src_dtype >= MXFP4_DT_BF16 && src_dtype <= MXFP4_DT_F32, "quantize: bad dtype %d", src_dtype);
    MXH_REQUIRE(((uintptr_t)q & 3) == 0, "quantize: packed output must be 4-byte aligned");
    if (M == 0 || Kp == 0) return MXFP4_OK;
    const int esz = src_dtype == MXFP4_DT_F32 ? 4 : 2;
    const int vec = (((uintptr_t)x & 15) == 0) && ((ldx * esz) % 16 == 0);
    MXH_REQUIRE(round_to_f16 >= 0 && round_to_f16 <= 2, "quantize: rounding mode %d (0, 1 fp16, 2 bf16)", round_to_f16);
    if (src_dtype == MXFP4_DT_BF16) {
        // bf16 input is already bf16
        if (round_to_f16 == 1) launch_quant<MXFP4_DT_BF16, 1>(x, ldx, M, K, Kp, vec, q, s, st);
        else launch_quant<MXFP4_DT_BF16, 0>(x, ldx, M, K, Kp, vec, q, s, st);
    } else if (src_dtype == MXFP4_DT_F16) {
        if (round_to_f16 == 2) launch_quant<MXFP4_DT_F16, 2>(x, ldx, M, K, Kp, vec, q, s, st);
        else launch_quant<MXFP4_DT_F16, 0>(x, ldx, M, K, Kp, vec, q, s, st);
    } else {
        if (round_to_f16 == 1) launch_quant<MXFP4_DT_F32, 1>(x, ldx, M, K, Kp, vec, q, s, st);
        else if (round_to_f16 == 2) launch_quant<MXFP4_DT_F32, 2>(x, ldx, M, K, Kp, vec, q, s, st);
        else launch_quant<MXFP4_DT_F32, 0>(x, ldx, M, K, Kp, vec, q, s, st);
    }
    return launch_status("quantize_rows");
}
}  // namespace mxh

extern "C" int mxfp4_quantize_rows(const void* x, int src_dtype, int round_to_f16, int64_t ldx, int M,
                                   int K, int Kp, uint8_t* q, uint8_t* s, void* stream) {
    return mxh::quantize_rows_impl(x, src_dtype, round_to_f16, ldx, M, K, Kp, q, s, mxh::as_stream(stream));
}

extern "C" int mxfp4_prequant(const void* x, int64_t ldx, int M, int K, int Kp, uint8_t* xq,
                              uint8_t* xsc, void* stream) {
    return mxh::quantize_rows_impl(x, MXFP4_DT_BF16, 0, ldx, M, K, Kp, xq, xsc, mxh::as_stream(stream));
}
