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
#include "mx_device.h"
#include "mx_host.h"
#include "kv_codec.h"

namespace {

using kv::e4m3_ref_decode;
using kv::e4m3_ref_encode;

constexpr int kD = 128;          // head dimension (the reference's kernels assume 128)
constexpr int kChunk = 64;       // positions per score workgroup

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

constexpr int kPart = 132;       // floats per partial record: max, sum, 128 column sums, pad
constexpr int kMaxChunks = 1024; // max_pos <= 65536

// Workgroup (64-position chunk, kv head g, token m):
//  1. the chunk's K and V rows and the group's q are loaded before anything
//     waits (the position only masks; rows past max_pos are clamped), so the
//     workgroup pays one memory latency;
//  2. scores of all G query heads of the group (raw dot products also go to
//     sc), per head the chunk max, exp(x - max) and sum, and the partial
//     weighted sum of V -> one record per (token, head, chunk).
template <int G>
__global__ __launch_bounds__(256) void attn_partial_kernel(const uint16_t* __restrict__ q,
                                                           const uint8_t* __restrict__ kvk,
                                                           const uint8_t* __restrict__ kvv, float* __restrict__ sc,
                                                           float* __restrict__ part, const int32_t* __restrict__ dpos,
                                                           int Hq, int Hkv, int max_pos, int nchunk, float invsqrt) {
    const int m = blockIdx.z, g = blockIdx.y, chunk = blockIdx.x;
    const int tid = threadIdx.x;
    const int s0 = chunk * kChunk;
    const int rowmax = max_pos - 1 - s0;       // last in-bounds row of the chunk (s0 < max_pos)
    __shared__ __align__(16) float qs[G][kD];
    __shared__ float ps[G][kChunk];
    __shared__ __align__(16) float vred[8][G][kD];   // V partial sums of the 8 position lanes
    __shared__ float stat[G][2];
    // ---- 1. loads: K words of the score thread (position p, quarter qd of
    // D), V words of the partial-sum thread (4 columns cq, positions
    // pl*8..pl*8+7), 4 q values per thread
    const int p = tid >> 2, qd = tid & 3;
    const uint8_t* kr = kvk + ((int64_t)(s0 + min(p, rowmax)) * Hkv + g) * kD + qd * 32;
    const uint4 b0 = *reinterpret_cast<const uint4*>(kr);
    const uint4 b1 = *reinterpret_cast<const uint4*>(kr + 16);
    const int cq = tid & 31, pl = tid >> 5;
    uint32_t vw[8];
    {
        const uint8_t* vcol = kvv + ((int64_t)s0 * Hkv + g) * kD + cq * 4;
        const int64_t vstride = (int64_t)Hkv * kD;
#pragma unroll
        for (int i = 0; i < 8; ++i) vw[i] = *reinterpret_cast<const uint32_t*>(vcol + (int64_t)min(pl * 8 + i, rowmax) * vstride);
    }
    constexpr int kQPer = (G * kD + 1023) / 1024;    // 4-value q loads per thread
    uint2 qv[kQPer];
#pragma unroll
    for (int j = 0; j < kQPer; ++j) {
        const int i = (j * 256 + tid) * 4;
        qv[j] = i < G * kD ? *reinterpret_cast<const uint2*>(q + ((int64_t)m * Hq + g * G) * kD + i) : make_uint2(0, 0);
    }
    const int pos = *dpos + m;
    if (pos < 0 || pos >= max_pos) return;
    const int S = pos + 1;
    if (s0 >= S) return;                       // uniform over the workgroup; not counted below
    const int s = s0 + p;
#pragma unroll
    for (int j = 0; j < kQPer; ++j) {
        const int i = (j * 256 + tid) * 4;
        if (i < G * kD) {
            float* d = &qs[0][0] + i;
            d[0] = bf16_to_f32(qv[j].x & 0xFFFFu);
            d[1] = bf16_to_f32(qv[j].x >> 16);
            d[2] = bf16_to_f32(qv[j].y & 0xFFFFu);
            d[3] = bf16_to_f32(qv[j].y >> 16);
        }
    }
    __syncthreads();
    // ---- 2a. scores
    {
        float acc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h] = 0.0f;
        if (s < S) {
            const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            // 4 columns per step: their q values come from LDS as one float4
            // per head (the 16 threads of a quarter read the same address)
#pragma unroll 2
            for (int jj = 0; jj < 8; ++jj) {
                uint32_t wj = w[0];   // w[jj] by selects: no dynamic register index
#pragma unroll
                for (int t = 1; t < 8; ++t) wj = jj == t ? w[t] : wj;
                const float k0 = e4m3_ref_decode(wj & 0xFFu), k1 = e4m3_ref_decode((wj >> 8) & 0xFFu);
                const float k2 = e4m3_ref_decode((wj >> 16) & 0xFFu), k3 = e4m3_ref_decode(wj >> 24);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    const float4 qf = *reinterpret_cast<const float4*>(&qs[h][qd * 32 + jj * 4]);
                    acc[h] = fmaf(qf.x, k0, fmaf(qf.y, k1, fmaf(qf.z, k2, fmaf(qf.w, k3, acc[h]))));
                }
            }
        }
        // sum the four quarters of D (lanes of a quad)
#pragma unroll
        for (int h = 0; h < G; ++h) {
            acc[h] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[h]), 0xB1, 0xF, 0xF, true));
            acc[h] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[h]), 0x4E, 0xF, 0xF, true));
        }
        if (qd == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                if (s < S) sc[((int64_t)m * Hq + g * G + h) * max_pos + s] = acc[h];
                ps[h][p] = s < S ? acc[h] * invsqrt : -INFINITY;
            }
        }
    }
    __syncthreads();
    // ---- 2b. per head: chunk max, exp, sum (32 threads per head, 2 positions each)
    {
        const int j = tid & 31;
        for (int h = tid >> 5; h < G; h += 8) {
            const float x0 = ps[h][j], x1 = ps[h][j + 32];
            float mx = fmaxf(x0, x1);
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 32));
            const float e0 = expf(x0 - mx), e1 = expf(x1 - mx);   // exp(-inf) = 0 past S
            ps[h][j] = e0;
            ps[h][j + 32] = e1;
            float l = e0 + e1;
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) l += __shfl_xor(l, off, 32);
            if (j == 0) {
                stat[h][0] = mx;
                stat[h][1] = l;
            }
        }
    }
    __syncthreads();
    // ---- 2c. partial V sums: thread = 4 columns (cq) x 8 of the chunk's
    // positions (pl), all G heads; rows past S carry weight 0 (their bytes
    // decode to finite values).  The 8 position lanes are summed through LDS.
    {
        float4 acc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float v0 = e4m3_ref_decode(vw[i] & 0xFFu), v1 = e4m3_ref_decode((vw[i] >> 8) & 0xFFu);
            const float v2 = e4m3_ref_decode((vw[i] >> 16) & 0xFFu), v3 = e4m3_ref_decode(vw[i] >> 24);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float w = ps[h][pl * 8 + i];
                acc[h].x = fmaf(w, v0, acc[h].x);
                acc[h].y = fmaf(w, v1, acc[h].y);
                acc[h].z = fmaf(w, v2, acc[h].z);
                acc[h].w = fmaf(w, v3, acc[h].w);
            }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) *reinterpret_cast<float4*>(&vred[pl][h][cq * 4]) = acc[h];
        __syncthreads();
        for (int i = tid; i < G * kD; i += 256) {
            const int h = i / kD, col = i % kD;
            float sum = 0.0f;
#pragma unroll
            for (int l = 0; l < 8; ++l) sum += vred[l][h][col];
            float* rec = part + (((int64_t)m * Hq + g * G + h) * nchunk + chunk) * kPart;
            rec[4 + col] = sum;
            if (col == 0) {
                rec[0] = stat[h][0];
                rec[1] = stat[h][1];
            }
        }
    }
}

// Workgroup (query head h, token m), 256 threads: merges the chunk records,
// o = sum_c exp(m_c - M) acc_c / sum_c exp(m_c - M) l_c with M = max_c m_c.
// Pass 1 loads every chunk's (m_c, l_c) at once (a thread per chunk); pass 2
// has thread (column pair cp, chunk phase cq) sum the chunks c = cq mod 4
// with all of its loads in flight, and the four phases meet in LDS.  The
// output is fp32 o and/or the MXFP4 rows (oq, os) of bf16(o) (32-blocks of
// 16 column pairs, the quantizer's rule).
__global__ __launch_bounds__(256) void attn_final_kernel(const float* __restrict__ part, float* __restrict__ o,
                                                         uint8_t* __restrict__ oq, uint8_t* __restrict__ os,
                                                         const int32_t* __restrict__ dpos, int Hq, int max_pos,
                                                         int nchunk) {
    const int h = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const int pos = *dpos + m;
    if (pos < 0 || pos >= max_pos) return;
    const int n = pos / kChunk + 1;            // chunks holding positions 0..pos
    const float* rec = part + ((int64_t)m * Hq + h) * nchunk * kPart;
    __shared__ float cw[kMaxChunks];           // chunk max, then its weight exp(m_c - M)
    __shared__ float red[4];
    __shared__ __align__(8) float2 nred[4][64];
    constexpr int kPer = kMaxChunks / 256;
    float mc[kPer], lc[kPer];
    float gm = -INFINITY;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int c = i * 256 + tid;
        mc[i] = -INFINITY;
        lc[i] = 0.0f;
        if (c < n) {
            const float2 st = *reinterpret_cast<const float2*>(rec + (int64_t)c * kPart);
            mc[i] = st.x;
            lc[i] = st.y;
        }
        gm = fmaxf(gm, mc[i]);
    }
    const int lane = tid & 63, wave = tid >> 6;
    gm = mx::wave_reduce_dpp<true>(gm);
    if (lane == 0) red[wave] = gm;
    __syncthreads();
    gm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float den = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int c = i * 256 + tid;
        if (c < n) {
            const float w = expf(mc[i] - gm);
            cw[c] = w;
            den = fmaf(w, lc[i], den);
        }
    }
    den = mx::wave_reduce_dpp<false>(den);
    __syncthreads();                           // red[] reads above are done
    if (lane == 0) red[wave] = den;
    __syncthreads();                           // cw[] and red[] complete
    den = (red[0] + red[1]) + (red[2] + red[3]);
    // pass 2: thread = (column pair cp = lane, phase cq = wave)
    float2 num = make_float2(0.0f, 0.0f);
    const float* colp = rec + 4 + 2 * lane;
#pragma unroll 16
    for (int c = wave; c < n; c += 4) {
        const float2 a = *reinterpret_cast<const float2*>(colp + (int64_t)c * kPart);
        const float w = cw[c];
        num.x = fmaf(w, a.x, num.x);
        num.y = fmaf(w, a.y, num.y);
    }
    nred[wave][lane] = num;
    __syncthreads();
    if (wave != 0) return;
    num.x = (nred[0][lane].x + nred[1][lane].x) + (nred[2][lane].x + nred[3][lane].x);
    num.y = (nred[0][lane].y + nred[1][lane].y) + (nred[2][lane].y + nred[3][lane].y);
    const float r0 = num.x / den, r1 = num.y / den;
    if (o) *reinterpret_cast<float2*>(o + ((int64_t)m * Hq + h) * kD + 2 * lane) = make_float2(r0, r1);
    if (oq) {
        // MXFP4 of bf16(o): a 32-block is 16 lanes; the quantizer's rule
        const float v0 = mx::bf16_to_f32(mx::f32_to_bf16_rne(r0));
        const float v1 = mx::bf16_to_f32(mx::f32_to_bf16_rne(r1));
        float am = fmaxf(__builtin_fabsf(v0), __builtin_fabsf(v1));
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) am = fmaxf(am, __shfl_xor(am, off));
        const uint32_t code = mx::e8m0_code(am);
        const float inv = mx::e8m0_inv_scale(code);
        uint32_t byte = mx::e2m1_code(v0 * inv) | (mx::e2m1_code(v1 * inv) << 4);
        byte |= (uint32_t)__shfl_down((int)byte, 1) << 8;
        byte |= (uint32_t)__shfl_down((int)byte, 2) << 16;
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

extern "C" int mxfp4_attn_decode_mx(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                                    float* sc, float* o, uint8_t* oq, uint8_t* os, int M, int Hq, int Hkv, int D,
                                    int max_pos, void* workspace, size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(q && kvk && kvv && dpos && sc && workspace, "attn_decode: null pointer");
    MXH_REQUIRE(o || oq, "attn_decode: no output (o and oq both null)");
    MXH_REQUIRE(!oq == !os, "attn_decode: oq and os go together");
    MXH_REQUIRE(D == kD, "attn_decode: head_dim D=%d (this build supports %d, as the reference's kernels)", D, kD);
    MXH_REQUIRE(M > 0 && M <= 65535 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "attn_decode: M=%d Hq=%d Hkv=%d", M, Hq, Hkv);
    MXH_REQUIRE(max_pos > 0 && max_pos <= kChunk * kMaxChunks, "attn_decode: max_pos=%d (1..%d)", max_pos,
                kChunk * kMaxChunks);
    MXH_REQUIRE(((uintptr_t)kvk & 15) == 0 && ((uintptr_t)kvv & 3) == 0, "attn_decode: kv cache rows must be aligned");
    MXH_REQUIRE(((uintptr_t)q & 7) == 0, "attn_decode: q must be 8-byte aligned");
    MXH_REQUIRE(!o || ((uintptr_t)o & 7) == 0, "attn_decode: o must be 8-byte aligned");
    MXH_REQUIRE(!oq || ((uintptr_t)oq & 3) == 0, "attn_decode: oq must be 4-byte aligned");
    MXH_REQUIRE(workspace_bytes >= mxfp4_attn_decode_workspace_size(M, Hq, max_pos) && ((uintptr_t)workspace & 15) == 0,
                "attn_decode: workspace must be 16-byte aligned and hold mxfp4_attn_decode_workspace_size bytes");
    const int G = Hq / Hkv;
    const int nchunk = (max_pos + kChunk - 1) / kChunk;
    const float invsqrt = 1.0f / sqrtf((float)D);
    hipStream_t st = mxh::as_stream(stream);
    const dim3 gp(nchunk, Hkv, M);
    const uint16_t* qh = static_cast<const uint16_t*>(q);
    float* part = static_cast<float*>(workspace);
#define MXH_ATTN(GG)                                                                                         \
    hipLaunchKernelGGL(attn_partial_kernel<GG>, gp, dim3(256), 0, st, qh, kvk, kvv, sc, part, dpos, Hq, Hkv, \
                       max_pos, nchunk, invsqrt)
    switch (G) {
        case 1: MXH_ATTN(1); break;
        case 2: MXH_ATTN(2); break;
        case 4: MXH_ATTN(4); break;
        case 8: MXH_ATTN(8); break;
        case 16: MXH_ATTN(16); break;
        default: MXH_REQUIRE(false, "attn_decode: Hq/Hkv=%d must be 1, 2, 4, 8 or 16", G);
    }
#undef MXH_ATTN
    const int rc = mxh::launch_status("attn_decode (partials)");
    if (rc != MXFP4_OK) return rc;
    hipLaunchKernelGGL(attn_final_kernel, dim3(Hq, M), dim3(256), 0, st, part, o, oq, os, dpos, Hq, max_pos, nchunk);
    return mxh::launch_status("attn_decode (merge)");
}

extern "C" int mxfp4_attn_decode(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                                 float* sc, float* o, int M, int Hq, int Hkv, int D, int max_pos, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(o, "attn_decode: null pointer");
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
