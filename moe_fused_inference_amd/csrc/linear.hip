// linear.hip -- C-ABI entry points of the block-scaled linear operators.
//
//   mxfp4_lin_pq          replaces src/ext/mxfp4_decode.cu:311-318 (lin_pq)
//   mxfp4_linear_forward  replaces src/ext/mxfp4_linear.cu:200-206 (forward)
//
// `forward` rounds the activations to fp16 (src/ext/mxfp4_binding.cpp:31),
// quantizes them once with the bit-exact quantizer into the caller's
// workspace (the reference re-quantizes every 32-block inside each of its
// N/32 column blocks, src/ext/mxfp4_linear.cu:129-155), then runs lin_pq.
#include "mx_device.h"
#include "mx_host.h"

namespace mxh {
int quantize_rows_impl(const void* x, int src_dtype, int round_to_f16, int64_t ldx, int M, int K,
                       int Kp, uint8_t* q, uint8_t* s, hipStream_t st);
int lin_pq_gemv(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc,
                float* y, int M, int N, int K, int Kp, hipStream_t st);
int lin_pq_gemm(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc,
                float* y, int M, int N, int Kp, hipStream_t st);
bool lin_pq_gemm_supported(int M, int N, int Kp);
int lin_pq_gemm2(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc,
                 float* y, int M, int N, int Kp, hipStream_t st);
bool lin_pq_gemm2_supported(int M, int N, int Kp);
}  // namespace mxh

namespace {
constexpr int kGemvMaxM = 16;  // up to one MFMA row tile: grouped GEMV
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

extern "C" int mxfp4_lin_pq(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc,
                            float* y, int M, int N, int K, int Kp, void* stream) {
    MXH_REQUIRE(xq && xsc && wp && wsc && y, "lin_pq: null pointer");
    MXH_REQUIRE(M > 0 && N > 0 && Kp > 0, "lin_pq: sizes must be positive (M=%d N=%d Kp=%d)", M, N, Kp);
    MXH_REQUIRE(Kp % 32 == 0, "lin_pq: Kp=%d must be a multiple of 32", Kp);
    MXH_REQUIRE(K <= Kp, "lin_pq: K=%d exceeds Kp=%d", K, Kp);
    hipStream_t st = mxh::as_stream(stream);
    if (M > kGemvMaxM && mxh::lin_pq_gemm2_supported(M, N, Kp))
        return mxh::lin_pq_gemm2(xq, xsc, wp, wsc, y, M, N, Kp, st);
    if (M > kGemvMaxM && mxh::lin_pq_gemm_supported(M, N, Kp))
        return mxh::lin_pq_gemm(xq, xsc, wp, wsc, y, M, N, Kp, st);
    return mxh::lin_pq_gemv(xq, xsc, wp, wsc, y, M, N, K, Kp, st);
}

extern "C" size_t mxfp4_linear_workspace_size(int M, int Kp) {
    if (M <= 0 || Kp <= 0) return 0;
    return align256((size_t)M * (Kp / 2)) + align256((size_t)M * (Kp / 32));
}

extern "C" int mxfp4_linear_forward(const void* x, int x_dtype, const uint8_t* wp, const uint8_t* wsc,
                                    float* y, int M, int N, int K, int Kp, void* workspace,
                                    size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(x && wp && wsc && y && workspace, "forward: null pointer");
    MXH_REQUIRE(x_dtype == MXFP4_DT_BF16 || x_dtype == MXFP4_DT_F16, "forward: x must be bf16 or fp16");
    MXH_REQUIRE(M > 0 && N > 0 && K > 0, "forward: sizes must be positive (M=%d N=%d K=%d)", M, N, K);
    MXH_REQUIRE(Kp % 32 == 0 && Kp >= K, "forward: Kp=%d must be a multiple of 32 and >= K=%d", Kp, K);
    const size_t need = mxfp4_linear_workspace_size(M, Kp);
    MXH_REQUIRE(workspace_bytes >= need, "forward: workspace %zu B < required %zu B", workspace_bytes, need);
    MXH_REQUIRE(((uintptr_t)workspace & 255) == 0, "forward: workspace must be 256-byte aligned");
    uint8_t* xq = static_cast<uint8_t*>(workspace);
    uint8_t* xsc = xq + align256((size_t)M * (Kp / 2));
    hipStream_t st = mxh::as_stream(stream);
    int rc = mxh::quantize_rows_impl(x, x_dtype, /*round_to_f16=*/1, K, M, K, Kp, xq, xsc, st);
    if (rc != MXFP4_OK) return rc;
    return mxfp4_lin_pq(xq, xsc, wp, wsc, y, M, N, K, Kp, stream);
}
