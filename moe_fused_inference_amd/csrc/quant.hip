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
#include "quant_rows.h"

namespace {

// Workgroup (row group blockIdx.x, unit segment blockIdx.y): 2^lt threads per
// row (the units of a row rounded up to a power of two, at most 256), so the
// row and unit of a thread are shifts and masks, not a division.
template <int SRC, int RND>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const void* __restrict__ x, int64_t ldx,
                                                            int M, int K, int Kp, int vec, int lt,
                                                            uint8_t* __restrict__ q,
                                                            uint8_t* __restrict__ s) {
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * (256 >> lt) + (tid >> lt);
    const int u = (int)blockIdx.y * (1 << lt) + (tid & ((1 << lt) - 1));
    mxq::quantize_unit<SRC, RND>(x, ldx, M, K, Kp, vec != 0, row, u, q, s);
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
