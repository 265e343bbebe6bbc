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
//                        (split softmax: rescale by exp(m_c - max)).
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

// Workgroup (64-position chunk, kv head g, token m): the scores of the chunk
// for all G query heads of the group (K rows read once, q staged in LDS),
// stored raw into sc; then per head the chunk's max, exp(x - max) and sum,
// and the partial weighted sum of the chunk's V rows (read once for the
// group).  Writes one partial record per (token, head, chunk).
template <int G>
__global__ __launch_bounds__(256) void attn_partial_kernel(const uint16_t* __restrict__ q,
                                                           const uint8_t* __restrict__ kvk,
                                                           const uint8_t* __restrict__ kvv, float* __restrict__ sc,
                                                           float* __restrict__ part, const int32_t* __restrict__ dpos,
                                                           int Hq, int Hkv, int max_pos, int nchunk, float invsqrt) {
    const int m = blockIdx.z, g = blockIdx.y, chunk = blockIdx.x;
    const int pos = *dpos + m;
    if (pos < 0 || pos >= max_pos) return;
    const int S = pos + 1;
    const int s0 = chunk * kChunk;
    if (s0 >= S) return;                       // uniform over the workgroup
    __shared__ __align__(16) float qs[G][kD];
    __shared__ float ps[G][kChunk];
    // Both phases' cache rows are loaded first (one memory latency for the
    // workgroup): K words of the score thread (position p, quarter qd of D)
    // and V words of the partial-sum thread (4 columns cq, positions
    // pl*8..pl*8+7; rows past S clamped in bounds, their weight is 0).
    const int p = threadIdx.x >> 2, qd = threadIdx.x & 3;
    const int s = s0 + p;
    uint4 b0 = make_uint4(0, 0, 0, 0), b1 = make_uint4(0, 0, 0, 0);
    if (s < S) {
        const uint8_t* kr = kvk + ((int64_t)s * Hkv + g) * kD + qd * 32;
        b0 = *reinterpret_cast<const uint4*>(kr);
        b1 = *reinterpret_cast<const uint4*>(kr + 16);
    }
    const int cq = threadIdx.x & 31, pl = threadIdx.x >> 5;
    const int last = S - 1 - s0;               // last valid row of the chunk
    uint32_t vw[8];
    {
        const uint8_t* vcol = kvv + ((int64_t)s0 * Hkv + g) * kD + cq * 4;
        const int64_t vstride = (int64_t)Hkv * kD;
#pragma unroll
        for (int i = 0; i < 8; ++i) vw[i] = *reinterpret_cast<const uint32_t*>(vcol + (int64_t)min(pl * 8 + i, last) * vstride);
    }
    for (int i = threadIdx.x; i < G * kD; i += 256)
        qs[i / kD][i % kD] = bf16_to_f32(q[((int64_t)m * Hq + g * G + i / kD) * kD + i % kD]);
    __syncthreads();
    // ---- scores: thread = (position p, quarter qd of D)
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
        if (qd == 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                if (s < S) sc[((int64_t)m * Hq + g * G + h) * max_pos + s] = acc[h];
                ps[h][p] = s < S ? acc[h] * invsqrt : -INFINITY;
            }
        }
    }
    __syncthreads();
    // ---- per head: chunk max, exp, sum (32 threads per head, 2 positions each)
    __shared__ float stat[G][2];
    {
        const int j = threadIdx.x & 31;
        for (int h = threadIdx.x >> 5; h < G; h += 8) {
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
    // ---- partial V sums: thread = 4 columns (cq) x 8 of the chunk's
    // positions (pl), all G heads, from the V words loaded at entry.  The 8
    // position lanes are summed through LDS.
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
        __shared__ __align__(16) float vred[8][G][kD];
#pragma unroll
        for (int h = 0; h < G; ++h) *reinterpret_cast<float4*>(&vred[pl][h][cq * 4]) = acc[h];
        __syncthreads();
        for (int i = threadIdx.x; i < G * kD; i += 256) {
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

// Workgroup (query head, token), thread = column: merges the chunk records,
// o = sum_c exp(m_c - M) acc_c / sum_c exp(m_c - M) l_c with M = max_c m_c.
// The chunk statistics are loaded in parallel (a thread per chunk) and the
// column sums with many loads in flight.
constexpr int kMaxChunks = 1024;   // max_pos <= 65536
__global__ __launch_bounds__(128) void attn_final_kernel(const float* __restrict__ part, float* __restrict__ o,
                                                         const int32_t* __restrict__ dpos, int Hq, int max_pos,
                                                         int nchunk) {
    const int h = blockIdx.x, m = blockIdx.y, c = threadIdx.x;
    const int pos = *dpos + m;
    if (pos < 0 || pos >= max_pos) return;
    const int n = pos / kChunk + 1;            // chunks holding positions 0..pos
    const float* rec = part + ((int64_t)m * Hq + h) * nchunk * kPart;
    __shared__ float cw[kMaxChunks];           // chunk max, then its scale exp(m_c - M)
    __shared__ float red[2];
    float gm = -INFINITY;
    for (int i = c; i < n; i += kD) {
        cw[i] = rec[(int64_t)i * kPart];
        gm = fmaxf(gm, cw[i]);
    }
    gm = mx::wave_reduce_dpp<true>(gm);
    if ((c & 63) == 0) red[c >> 6] = gm;
    __syncthreads();
    gm = fmaxf(red[0], red[1]);
    float dpart = 0.0f;
    for (int i = c; i < n; i += kD) {
        const float w = expf(cw[i] - gm);
        cw[i] = w;
        dpart = fmaf(w, rec[(int64_t)i * kPart + 1], dpart);
    }
    dpart = mx::wave_reduce_dpp<false>(dpart);
    __syncthreads();                           // red[] reads above are done
    if ((c & 63) == 0) red[c >> 6] = dpart;
    __syncthreads();
    const float den = red[0] + red[1];
    float num = 0.0f;
    const float* col = rec + 4 + c;
#pragma unroll 16
    for (int i = 0; i < n; ++i) num = fmaf(cw[i], col[(int64_t)i * kPart], num);
    o[((int64_t)m * Hq + h) * kD + c] = num / den;
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

extern "C" int mxfp4_attn_decode(const void* q, const uint8_t* kvk, const uint8_t* kvv, const int32_t* dpos,
                                 float* sc, float* o, int M, int Hq, int Hkv, int D, int max_pos, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(q && kvk && kvv && dpos && sc && o && workspace, "attn_decode: null pointer");
    MXH_REQUIRE(D == kD, "attn_decode: head_dim D=%d (this build supports %d, as the reference's kernels)", D, kD);
    MXH_REQUIRE(M > 0 && M <= 65535 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "attn_decode: M=%d Hq=%d Hkv=%d", M, Hq, Hkv);
    MXH_REQUIRE(max_pos > 0 && max_pos <= kChunk * kMaxChunks, "attn_decode: max_pos=%d (1..%d)", max_pos,
                kChunk * kMaxChunks);
    MXH_REQUIRE(((uintptr_t)kvk & 15) == 0 && ((uintptr_t)kvv & 3) == 0, "attn_decode: kv cache rows must be aligned");
    MXH_REQUIRE(workspace_bytes >= mxfp4_attn_decode_workspace_size(M, Hq, max_pos) && ((uintptr_t)workspace & 15) == 0,
                "attn_decode: workspace must be 16-byte aligned and hold mxfp4_attn_decode_workspace_size bytes");
    const int G = Hq / Hkv;
    const int nchunk = (max_pos + kChunk - 1) / kChunk;
    const float invsqrt = 1.0f / sqrtf((float)D);
    hipStream_t st = mxh::as_stream(stream);
    const dim3 gp(nchunk, Hkv, M);
    const uint16_t* qh = static_cast<const uint16_t*>(q);
    float* part = static_cast<float*>(workspace);
#define MXH_ATTN_PARTIAL(GG)                                                                                          \
    hipLaunchKernelGGL(attn_partial_kernel<GG>, gp, dim3(256), 0, st, qh, kvk, kvv, sc, part, dpos, Hq, Hkv, max_pos, \
                       nchunk, invsqrt)
    switch (G) {
        case 1: MXH_ATTN_PARTIAL(1); break;
        case 2: MXH_ATTN_PARTIAL(2); break;
        case 4: MXH_ATTN_PARTIAL(4); break;
        case 8: MXH_ATTN_PARTIAL(8); break;
        case 16: MXH_ATTN_PARTIAL(16); break;
        default: MXH_REQUIRE(false, "attn_decode: Hq/Hkv=%d must be 1, 2, 4, 8 or 16", G);
    }
#undef MXH_ATTN_PARTIAL
    const int rc = mxh::launch_status("attn_decode (partials)");
    if (rc != MXFP4_OK) return rc;
    hipLaunchKernelGGL(attn_final_kernel, dim3(Hq, M), dim3(kD), 0, st, part, o, dpos, Hq, max_pos, nchunk);
    return mxh::launch_status("attn_decode (merge)");
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
