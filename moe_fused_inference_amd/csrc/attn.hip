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
//   attn_score_kernel    workgroup (64 positions, kv head g, token m): the
//                        K rows are read once for all G query heads of the
//                        group (q staged in LDS); thread = (position,
//                        quarter of D); raw dot products go to sc (M, Hq,
//                        max_pos), the scratch the reference's interface
//                        hands over.
//   attn_combine_kernel  workgroup (query head, token): max and sum of
//                        score/sqrt(D) over the positions, then the weighted
//                        sum of the V rows (thread = 4 columns x one of 8
//                        position lanes), o = acc / sum.
//   kv_write_kernel      k, v (M, Hkv, D) bf16 -> E4M3 bytes at row pos.
//
// The byte codec is the reference's own (f32_to_e4m3 / e4m3_to_f32 at
// src/ext/mxfp4_decode.cu:355-364,437-455), kept exactly because caches and
// outputs must match it: rounding half away from zero, |v| >= 248 saturating
// to 0x7F, subnormal codes read as m * 2^-6 (standard E4M3: m * 2^-9) and
// exponent-15 codes read as 56 * (8 + m).
#include "mx_device.h"
#include "mx_host.h"

namespace {

constexpr int kD = 128;          // head dimension (the reference's kernels assume 128)
constexpr int kChunk = 64;       // positions per score workgroup

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

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

template <int G>
__global__ __launch_bounds__(256) void attn_score_kernel(const uint16_t* __restrict__ q, const uint8_t* __restrict__ kvk,
                                                         float* __restrict__ sc, const int32_t* __restrict__ dpos,
                                                         int Hq, int Hkv, int max_pos) {
    const int m = blockIdx.z, g = blockIdx.y;
    const int pos = *dpos + m;
    if (pos < 0 || pos >= max_pos) return;
    const int S = pos + 1;
    const int s0 = blockIdx.x * kChunk;
    if (s0 >= S) return;                       // uniform over the workgroup
    __shared__ __align__(16) float qs[G][kD];
    for (int i = threadIdx.x; i < G * kD; i += 256)
        qs[i / kD][i % kD] = bf16_to_f32(q[((int64_t)m * Hq + g * G + i / kD) * kD + i % kD]);
    __syncthreads();
    const int p = threadIdx.x >> 2, qd = threadIdx.x & 3;
    const int s = s0 + p;
    float acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h] = 0.0f;
    if (s < S) {
        const uint8_t* kr = kvk + ((int64_t)s * Hkv + g) * kD + qd * 32;
        const uint4 b0 = *reinterpret_cast<const uint4*>(kr);
        const uint4 b1 = *reinterpret_cast<const uint4*>(kr + 16);
        const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        // 4 columns per step: their q values come from LDS as one float4 per
        // head (the 16 threads of a quarter read the same address)
#pragma unroll 2
        for (int jj = 0; jj < 8; ++jj) {
            uint32_t wj = w[0];
#pragma unroll
            for (int t = 1; t < 8; ++t) wj = jj == t ? w[t] : wj;
            const float k0 = e4m3_ref_decode(wj & 0xFFu), k1 = e4m3_ref_decode((wj >> 8) & 0xFFu);
            const float k2 = e4m3_ref_decode((wj >> 16) & 0xFFu), k3 = e4m3_ref_decode(wj >> 24);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float4 qv = *reinterpret_cast<const float4*>(&qs[h][qd * 32 + jj * 4]);
                acc[h] = fmaf(qv.x, k0, fmaf(qv.y, k1, fmaf(qv.z, k2, fmaf(qv.w, k3, acc[h]))));
            }
        }
    }
    // sum the four quarters of D (lanes of a quad)
#pragma unroll
    for (int h = 0; h < G; ++h) {
        acc[h] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[h]), 0xB1, 0xF, 0xF, true));
        acc[h] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[h]), 0x4E, 0xF, 0xF, true));
    }
    if (s < S && qd == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) sc[((int64_t)m * Hq + g * G + h) * max_pos + s] = acc[h];
    }
}

__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ sc, const uint8_t* __restrict__ kvv,
                                                           float* __restrict__ o, const int32_t* __restrict__ dpos,
                                                           int Hq, int Hkv, int G, int max_pos, float invsqrt) {
    const int h = blockIdx.x, m = blockIdx.y;
    const int pos = *dpos + m;
    if (pos < 0 || pos >= max_pos) return;
    const int S = pos + 1;
    const int g = h / G;
    const float* srow = sc + ((int64_t)m * Hq + h) * max_pos;
    __shared__ float red[8][kD + 1];
    __shared__ float wred[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // max of score * invsqrt
    float smax = -INFINITY;
    for (int s = threadIdx.x; s < S; s += 256) smax = fmaxf(smax, srow[s] * invsqrt);
    smax = mx::wave_reduce_dpp<true>(smax);
    if (lane == 0) wred[wave] = smax;
    __syncthreads();
    smax = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
    // weighted V: thread = 4 columns (cq) x position lane pl
    const int cq = threadIdx.x & 31, pl = threadIdx.x >> 5;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, l = 0.f;
    const uint8_t* vcol = kvv + (int64_t)g * kD + cq * 4;
    const int64_t vstride = (int64_t)Hkv * kD;
    for (int s = pl; s < S; s += 8) {
        const float w = expf(srow[s] * invsqrt - smax);
        const uint32_t vb = *reinterpret_cast<const uint32_t*>(vcol + s * vstride);
        l += w;
        a0 = fmaf(w, e4m3_ref_decode(vb & 0xFFu), a0);
        a1 = fmaf(w, e4m3_ref_decode((vb >> 8) & 0xFFu), a1);
        a2 = fmaf(w, e4m3_ref_decode((vb >> 16) & 0xFFu), a2);
        a3 = fmaf(w, e4m3_ref_decode(vb >> 24), a3);
    }
    red[pl][cq * 4 + 0] = a0;
    red[pl][cq * 4 + 1] = a1;
    red[pl][cq * 4 + 2] = a2;
    red[pl][cq * 4 + 3] = a3;
    if (cq == 0) red[pl][kD] = l;
    __syncthreads();
    if (threadIdx.x < kD) {
        float acc = 0.f, den = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            acc += red[i][threadIdx.x];
            den += red[i][kD];
        }
        o[((int64_t)m * Hq + h) * kD + threadIdx.x] = acc / den;
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

extern "C" int mxfp4_attn_decode(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                                 float* sc, float* o, int M, int Hq, int Hkv, int D, int max_pos, void* stream) {
    MXH_REQUIRE(q && kvk && kvv && dpos && sc && o, "attn_decode: null pointer");
    MXH_REQUIRE(D == kD, "attn_decode: head_dim D=%d (this build supports %d, as the reference's kernels)", D, kD);
    MXH_REQUIRE(M > 0 && M <= 65535 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "attn_decode: M=%d Hq=%d Hkv=%d", M, Hq, Hkv);
    MXH_REQUIRE(max_pos > 0, "attn_decode: max_pos=%d", max_pos);
    MXH_REQUIRE(((uintptr_t)kvk & 15) == 0 && ((uintptr_t)kvv & 3) == 0, "attn_decode: kv cache rows must be aligned");
    const int G = Hq / Hkv;
    hipStream_t st = mxh::as_stream(stream);
    const dim3 gs((max_pos + kChunk - 1) / kChunk, Hkv, M);
    const uint16_t* qh = static_cast<const uint16_t*>(q);
    switch (G) {
        case 1: hipLaunchKernelGGL(attn_score_kernel<1>, gs, dim3(256), 0, st, qh, kvk, sc, dpos, Hq, Hkv, max_pos); break;
        case 2: hipLaunchKernelGGL(attn_score_kernel<2>, gs, dim3(256), 0, st, qh, kvk, sc, dpos, Hq, Hkv, max_pos); break;
        case 4: hipLaunchKernelGGL(attn_score_kernel<4>, gs, dim3(256), 0, st, qh, kvk, sc, dpos, Hq, Hkv, max_pos); break;
        case 8: hipLaunchKernelGGL(attn_score_kernel<8>, gs, dim3(256), 0, st, qh, kvk, sc, dpos, Hq, Hkv, max_pos); break;
        case 16: hipLaunchKernelGGL(attn_score_kernel<16>, gs, dim3(256), 0, st, qh, kvk, sc, dpos, Hq, Hkv, max_pos); break;
        default: MXH_REQUIRE(false, "attn_decode: Hq/Hkv=%d must be 1, 2, 4, 8 or 16", G);
    }
    const int rc = mxh::launch_status("attn_decode (scores)");
    if (rc != MXFP4_OK) return rc;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(Hq, M), dim3(256), 0, st, sc, kvv, o, dpos, Hq, Hkv, G, max_pos,
                       1.0f / sqrtf((float)D));
    return mxh::launch_status("attn_decode (combine)");
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
