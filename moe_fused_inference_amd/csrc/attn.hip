// attn.hip -- decode attention over an FP8 (E4M3) KV cache and the KV write,
// the remaining two ops of the reference's decode extension
// (src/ext/mxfp4_decode.cu:352-490, bound as attn_decode / kv_write in
// src/ext/mxfp4_decode_binding.cpp:161-173,213-230; called by
// runtime/model_runner_v2.py:256-260 and runtime/model_runner_v3.py:98-126).
//
// Token m (of M) sits at position pos = *dpos + m (read on the device, so a
// captured graph can advance it) and attends to positions 0..pos of one layer's
// cache kvk / kvv (max_pos, Hkv, D) bytes; q (M, Hq, D) bf16, Hq = G*Hkv (GQA).
//
//   attn_partial_kernel  workgroup (64 positions, kv head g, token m): the
//                        scores of the chunk for all G query heads of the
//                        group (K rows read once, q staged in LDS; the raw
//                        dot products also go to sc (M, Hq, max_pos), the
//                        scratch the reference's interface hands over), the
//                        chunk's softmax statistics and its partial weighted
//                        sum of V (V rows read once for the group) -> one
//                        record per (token, head, chunk) in the workspace.
//   attn_final_kernel    workgroup (query head, token): merges the records
//                        (split softmax: rescale by exp(m_c - max)); fp32
//                        output and/or its bf16 -> MXFP4 rows.
//   kv_write_kernel      k, v (M, Hkv, D) bf16 -> E4M3 bytes at row pos.
//
// The byte codec is the reference's own (f32_to_e4m3 / e4m3_to_f32 at
// src/ext/mxfp4_decode.cu:355-364,437-455), kept exactly because caches and
// outputs must match it: rounding half away from zero, |v| >= 248 saturating
// to 0x7F, subnormal codes read as m * 2^-6 (standard E4M3: m * 2^-9) and
// exponent-15 codes read as 56 * (8 + m).
#include "attn_merge.h"
#include "attn_partial.h"
#include "head_rope.h"
#include "mx_device.h"
#include "mx_host.h"
#include "kv_codec.h"

namespace {

using ap::kMaxFusedM;
using ap::QkvIn;
using kv::e4m3_ref_encode;

using am::kD;           // head dimension
using am::kChunk;       // positions per score workgroup

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

using am::kPart;        // floats per partial record: max, sum, 128 column sums, pad
using am::kMaxChunks;   // max_pos <= 65536

// The chunk pass (ap::attn_partial_body): workgroup (chunk, kv head g, token group).
template <int G, int RT, bool FUSED>
__global__ __launch_bounds__(256) void attn_partial_kernel(const uint16_t* __restrict__ q, const uint8_t* kvk,
                                                           const uint8_t* kvv, float* __restrict__ sc,
                                                           float* __restrict__ part, const int32_t* __restrict__ dpos,
                                                           int M, int Hq, int Hkv, int max_pos, int nchunk,
                                                           float invsqrt, QkvIn fz) {
    __shared__ ap::AttnLds<RT, FUSED> lds;
    ap::attn_partial_body<G, RT, FUSED>(lds, ap::PlainQkv{fz.qkv}, (int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z,
                                        q, kvk, kvv, sc, part, dpos, M, Hq, Hkv, max_pos, nchunk, invsqrt, fz);
}

// Workgroup (query head h, token m), 256 threads: merges the chunk records
// (am::merge_head).  The output is fp32 o and/or the MXFP4 rows (oq, os) of
// bf16(o) (32-blocks of 16 column pairs, the quantizer's rule).
__global__ __launch_bounds__(256) void attn_final_kernel(const float* __restrict__ part, float* __restrict__ o,
                                                         uint8_t* __restrict__ oq, uint8_t* __restrict__ os,
                                                         const int32_t* __restrict__ dpos, int Hq, int max_pos,
                                                         int nchunk) {
    const int h = blockIdx.x, m = blockIdx.y, lane = threadIdx.x & 63;
    const int pos = *dpos + m;
    if (pos < 0 || pos >= max_pos) return;
    const int n = pos / kChunk + 1;            // chunks holding positions 0..pos
    const float* rec = part + ((int64_t)m * Hq + h) * nchunk * kPart;
    __shared__ am::MergeLds lds;
    float r0, r1;
    if (!am::merge_head(rec, n, lds, r0, r1)) return;
    if (o) *reinterpret_cast<float2*>(o + ((int64_t)m * Hq + h) * kD + 2 * lane) = make_float2(r0, r1);
    if (oq) {
        uint32_t byte, code;
        am::quant_head_row(r0, r1, byte, code);
        const int64_t rowq = (int64_t)m * (Hq * kD / 2) + h * (kD / 2);
        if ((lane & 3) == 0) *reinterpret_cast<uint32_t*>(oq + rowq + lane) = byte;
        if ((lane & 15) == 0) os[(int64_t)m * (Hq * kD / 32) + h * (kD / 32) + lane / 16] = (uint8_t)code;
    }
}

__global__ __launch_bounds__(256) void kv_write_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                       uint8_t* __restrict__ kvk, uint8_t* __restrict__ kvv,
                                                       const int32_t* __restrict__ dpos, int M, int row_elems,
                                                       int max_pos) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int base = *dpos;
    if (base < 0 || idx >= (int64_t)M * row_elems) return;
    const int m = (int)(idx / row_elems);
    const int t = (int)(idx - (int64_t)m * row_elems);
    const int pos = base + m;
    if (pos >= max_pos) return;
    const int64_t off = (int64_t)pos * row_elems + t;
    kvk[off] = (uint8_t)e4m3_ref_encode(bf16_to_f32(k[idx]));
    kvv[off] = (uint8_t)e4m3_ref_encode(bf16_to_f32(v[idx]));
}

}  // namespace

extern "C" size_t mxfp4_attn_decode_workspace_size(int M, int Hq, int max_pos) {
    if (M <= 0 || Hq <= 0 || max_pos <= 0) return 0;
    const int64_t nchunk = (max_pos + kChunk - 1) / kChunk;
    return (size_t)((int64_t)M * Hq * nchunk * kPart * sizeof(float));
}

namespace {

template <bool FUSED>
int launch_attn(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos, float* sc, float* o,
                uint8_t* oq, uint8_t* os, int M, int Hq, int Hkv, int D, int max_pos, void* workspace,
                size_t workspace_bytes, const QkvIn& fz, hipStream_t st, bool merge = true) {
    MXH_REQUIRE(kvk && kvv && dpos && workspace, "attn_decode: null pointer");   // sc may be null: no scores kept
    MXH_REQUIRE(o || oq || !merge, "attn_decode: no output (o and oq both null)");
    MXH_REQUIRE(!oq == !os, "attn_decode: oq and os go together");
    MXH_REQUIRE(D == kD, "attn_decode: head_dim D=%d (this build supports %d, as the reference's kernels)", D, kD);
    MXH_REQUIRE(M > 0 && M <= 65535 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "attn_decode: M=%d Hq=%d Hkv=%d", M, Hq, Hkv);
    MXH_REQUIRE(max_pos > 0 && max_pos <= kChunk * kMaxChunks, "attn_decode: max_pos=%d (1..%d)", max_pos,
                kChunk * kMaxChunks);
    MXH_REQUIRE(((uintptr_t)kvk & 15) == 0 && ((uintptr_t)kvv & 3) == 0, "attn_decode: kv cache rows must be aligned");
    MXH_REQUIRE(!o || ((uintptr_t)o & 7) == 0, "attn_decode: o must be 8-byte aligned");
    MXH_REQUIRE(!oq || ((uintptr_t)oq & 3) == 0, "attn_decode: oq must be 4-byte aligned");
    MXH_REQUIRE(workspace_bytes >= mxfp4_attn_decode_workspace_size(M, Hq, max_pos) && ((uintptr_t)workspace & 15) == 0,
                "attn_decode: workspace must be 16-byte aligned and hold mxfp4_attn_decode_workspace_size bytes");
    const int G = Hq / Hkv;
    const int nchunk = (max_pos + kChunk - 1) / kChunk;
    const float invsqrt = 1.0f / sqrtf((float)D);
    // row tiles of 16 query rows per workgroup, at most 2: more token groups
    // (workgroups) rather than more rows each -- 4 tiles halved the grid at
    // M = 8 and took 9 % longer
    const int rows = M * G;
    const int RT = rows <= 16 ? 1 : 2;
    const int MT = (16 * RT) / G > 0 ? (16 * RT) / G : 1;
    MXH_REQUIRE(16 * RT >= G, "attn_decode: G=%d exceeds the 32 query rows of a workgroup", G);
    const dim3 gp(nchunk, Hkv, (M + MT - 1) / MT);
    const uint16_t* qh = static_cast<const uint16_t*>(q);
    float* part = static_cast<float*>(workspace);
#define MXH_ATTN(GG, RR)                                                                                         \
    hipLaunchKernelGGL((attn_partial_kernel<GG, RR, FUSED>), gp, dim3(256), 0, st, qh, kvk, kvv, sc, part, dpos, M, \
                       Hq, Hkv, max_pos, nchunk, invsqrt, fz)
#define MXH_ATTN_G(GG)                  \
    switch (RT) {                       \
        case 1: MXH_ATTN(GG, 1); break; \
        default: MXH_ATTN(GG, 2); break; \
    }
    switch (G) {
        case 1: MXH_ATTN_G(1); break;
        case 2: MXH_ATTN_G(2); break;
        case 4: MXH_ATTN_G(4); break;
        case 8: MXH_ATTN_G(8); break;
        case 16: MXH_ATTN_G(16); break;
        default: MXH_REQUIRE(false, "attn_decode: Hq/Hkv=%d must be 1, 2, 4, 8 or 16", G);
    }
#undef MXH_ATTN_G
#undef MXH_ATTN
    const int rc = mxh::launch_status("attn_decode (partials)");
    if (rc != MXFP4_OK || !merge) return rc;
    hipLaunchKernelGGL(attn_final_kernel, dim3(Hq, M), dim3(256), 0, st, part, o, oq, os, dpos, Hq, max_pos, nchunk);
    return mxh::launch_status("attn_decode (merge)");
}

}  // namespace

extern "C" int mxfp4_attn_decode_mx(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                                    float* sc, float* o, uint8_t* oq, uint8_t* os, int M, int Hq, int Hkv, int D,
                                    int max_pos, void* workspace, size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(q, "attn_decode: null pointer");
    MXH_REQUIRE(((uintptr_t)q & 15) == 0, "attn_decode: q must be 16-byte aligned");
    return launch_attn<false>(q, kvk, kvv, dpos, sc, o, oq, os, M, Hq, Hkv, D, max_pos, workspace, workspace_bytes,
                              QkvIn{}, mxh::as_stream(stream));
}

extern "C" int mxfp4_attn_decode_fused(const float* qkv, const void* q_norm_w, const void* k_norm_w, float eps,
                                       float theta, uint8_t* kvk, uint8_t* kvv, const int32_t* dpos, float* sc,
                                       float* o, uint8_t* oq, uint8_t* os, int M, int Hq, int Hkv, int D, int max_pos,
                                       int codec, void* workspace, size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(qkv && q_norm_w && k_norm_w, "attn_decode_fused: null pointer");
    MXH_REQUIRE(codec == 0 || codec == 1, "attn_decode_fused: codec %d (0 kv_write's, 1 torch float8_e4m3fn)", codec);
    MXH_REQUIRE(M > 0 && M <= kMaxFusedM, "attn_decode_fused: M=%d (1..%d)", M, kMaxFusedM);
    const QkvIn fz{qkv, static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w), eps, theta,
                   codec, kvk, kvv};
    return launch_attn<true>(nullptr, kvk, kvv, dpos, sc, o, oq, os, M, Hq, Hkv, D, max_pos, workspace,
                             workspace_bytes, fz, mxh::as_stream(stream));
}

extern "C" int mxfp4_attn_decode(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                                 float* sc, float* o, int M, int Hq, int Hkv, int D, int max_pos, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(o && sc, "attn_decode: null pointer");
    return mxfp4_attn_decode_mx(q, kvk, kvv, dpos, sc, o, nullptr, nullptr, M, Hq, Hkv, D, max_pos, workspace,
                                workspace_bytes, stream);
}

extern "C" int mxfp4_kv_write(const void* k, const void* v, uint8_t* kvk, uint8_t* kvv, const int32_t* dpos, int M,
                              int Hkv, int D, int max_pos, void* stream) {
    MXH_REQUIRE(k && v && kvk && kvv && dpos, "kv_write: null pointer");
    MXH_REQUIRE(M > 0 && Hkv > 0 && D > 0 && max_pos > 0, "kv_write: M=%d Hkv=%d D=%d max_pos=%d", M, Hkv, D, max_pos);
    const int64_t row = (int64_t)Hkv * D;
    MXH_REQUIRE(row * M < (1ll << 31), "kv_write: M*Hkv*D too large");
    const int64_t n = row * M;
    hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, mxh::as_stream(stream),
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), kvk, kvv, dpos, M, (int)row,
                       max_pos);
    return mxh::launch_status("kv_write");
}

extern "C" int mxfp4_attn_decode_fused_partials(const float* qkv, const void* q_norm_w, const void* k_norm_w,
                                                float eps, float theta, uint8_t* kvk, uint8_t* kvv,
                                                const int32_t* dpos, int M, int Hq, int Hkv, int D, int max_pos,
                                                int codec, void* workspace, size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(qkv && q_norm_w && k_norm_w, "attn_decode_fused_partials: null pointer");
    MXH_REQUIRE(codec == 0 || codec == 1, "attn_decode_fused_partials: codec %d (0 kv_write's, 1 torch float8_e4m3fn)",
                codec);
    MXH_REQUIRE(M > 0 && M <= kMaxFusedM, "attn_decode_fused_partials: M=%d (1..%d)", M, kMaxFusedM);
    const QkvIn fz{qkv, static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w), eps, theta,
                   codec, kvk, kvv};
    return launch_attn<true>(nullptr, kvk, kvv, dpos, nullptr, nullptr, nullptr, nullptr, M, Hq, Hkv, D, max_pos,
                             workspace, workspace_bytes, fz, mxh::as_stream(stream), false);
}
