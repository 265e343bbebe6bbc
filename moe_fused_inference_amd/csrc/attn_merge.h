// attn_merge.h -- the split-softmax merge of decode attention's chunk records,
// shared by attn_final_kernel (attn.hip) and the decode layer launch that
// runs the merge in front of o_proj and the MoE (decode_layer.hip), so both
// produce the same bits.
//
// A chunk record (kPart floats) holds the chunk's score maximum m_c, its sum
// of exp(s - m_c) l_c and the 128 column sums of exp(s - m_c) V; the merge of
// the n chunks of one (token, head) is
//     o = sum_c exp(m_c - M) acc_c / sum_c exp(m_c - M) l_c,  M = max_c m_c
// (the reference's single pass over all positions, src/ext/mxfp4_decode.cu:
// 366-430, split over chunks).
#pragma once
#include "mx_device.h"

namespace am {

constexpr int kD = 128;          // head dimension (the reference's kernels assume 128)
constexpr int kChunk = 64;       // positions per score workgroup
constexpr int kPart = 132;       // floats per partial record: max, sum, 128 column sums, pad
constexpr int kMaxChunks = 1024; // max_pos <= 65536

struct MergeLds {
    float cw[kMaxChunks];        // chunk max, then its weight exp(m_c - M) (long contexts)
    float red[4];
    float dred[4];
    float2 nred[4][64];
};

// Workgroup of 256 threads merging the n records at rec (record c at rec +
// c*kPart).  Up to 64 chunks (context 4096): one pass, thread (column pair
// lane, chunk phase wave) loads the statistics and column sums of chunks
// wave, wave + 4, ... at once.  Longer contexts: pass 1 loads every chunk's
// (m_c, l_c) (a thread per chunk), pass 2 sums the column records with all
// loads in flight.  The four phases meet in LDS.  Returns true in wave 0,
// whose lane l then holds o[2l], o[2l+1] in r0, r1; the other waves return
// false and must not wait at a barrier afterwards.
__device__ __forceinline__ bool merge_head(const float* rec, int n, MergeLds& s, float& r0, float& r1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (n <= 64) {
        constexpr int kF = 16;
        float2 st[kF], cs[kF];
#pragma unroll
        for (int i = 0; i < kF; ++i) {
            const int c = wave + 4 * i;
            st[i] = make_float2(-INFINITY, 0.0f);
            cs[i] = make_float2(0.0f, 0.0f);
            if (c < n) {
                st[i] = *reinterpret_cast<const float2*>(rec + (int64_t)c * kPart);
                cs[i] = *reinterpret_cast<const float2*>(rec + (int64_t)c * kPart + 4 + 2 * lane);
            }
        }
        float gm = -INFINITY;
#pragma unroll
        for (int i = 0; i < kF; ++i) gm = fmaxf(gm, st[i].x);
        if (lane == 0) s.red[wave] = gm;
        __syncthreads();
        gm = fmaxf(fmaxf(s.red[0], s.red[1]), fmaxf(s.red[2], s.red[3]));
        float den = 0.0f;
        float2 num = make_float2(0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < kF; ++i) {
            if (wave + 4 * i < n) {
                const float w = expf(st[i].x - gm);
                den = fmaf(w, st[i].y, den);
                num.x = fmaf(w, cs[i].x, num.x);
                num.y = fmaf(w, cs[i].y, num.y);
            }
        }
        s.nred[wave][lane] = num;
        if (lane == 0) s.dred[wave] = den;
        __syncthreads();
        if (wave != 0) return false;
        den = (s.dred[0] + s.dred[1]) + (s.dred[2] + s.dred[3]);
        num.x = (s.nred[0][lane].x + s.nred[1][lane].x) + (s.nred[2][lane].x + s.nred[3][lane].x);
        num.y = (s.nred[0][lane].y + s.nred[1][lane].y) + (s.nred[2][lane].y + s.nred[3][lane].y);
        r0 = num.x / den;
        r1 = num.y / den;
        return true;
    }
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
    gm = mx::wave_reduce_dpp<true>(gm);
    if (lane == 0) s.red[wave] = gm;
    __syncthreads();
    gm = fmaxf(fmaxf(s.red[0], s.red[1]), fmaxf(s.red[2], s.red[3]));
    float den = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int c = i * 256 + tid;
        if (c < n) {
            const float w = expf(mc[i] - gm);
            s.cw[c] = w;
            den = fmaf(w, lc[i], den);
        }
    }
    den = mx::wave_reduce_dpp<false>(den);
    __syncthreads();                           // red[] reads above are done
    if (lane == 0) s.red[wave] = den;
    __syncthreads();                           // cw[] and red[] complete
    den = (s.red[0] + s.red[1]) + (s.red[2] + s.red[3]);
    // pass 2: thread = (column pair cp = lane, phase cq = wave)
    float2 num = make_float2(0.0f, 0.0f);
    const float* colp = rec + 4 + 2 * lane;
#pragma unroll 16
    for (int c = wave; c < n; c += 4) {
        const float2 a = *reinterpret_cast<const float2*>(colp + (int64_t)c * kPart);
        const float w = s.cw[c];
        num.x = fmaf(w, a.x, num.x);
        num.y = fmaf(w, a.y, num.y);
    }
    s.nred[wave][lane] = num;
    __syncthreads();
    if (wave != 0) return false;
    num.x = (s.nred[0][lane].x + s.nred[1][lane].x) + (s.nred[2][lane].x + s.nred[3][lane].x);
    num.y = (s.nred[0][lane].y + s.nred[1][lane].y) + (s.nred[2][lane].y + s.nred[3][lane].y);
    r0 = num.x / den;
    r1 = num.y / den;
    return true;
}

// MXFP4 of bf16(o) for one head row held as merge_head leaves it (lane l:
// columns 2l, 2l+1): a 32-block is 16 lanes; the quantizer's rule.  Lane 4j
// receives the packed bytes of columns 8j .. 8j+7 (4 bytes, LSB first) in
// bytes4, and every lane its block's E8M0 code.  Wave 0, all 64 lanes.
__device__ __forceinline__ void quant_head_row(float r0, float r1, uint32_t& bytes4, uint32_t& code) {
    const float v0 = mx::bf16_to_f32(mx::f32_to_bf16_rne(r0));
    const float v1 = mx::bf16_to_f32(mx::f32_to_bf16_rne(r1));
    const float amax = mx::row16_reduce<true>(fmaxf(__builtin_fabsf(v0), __builtin_fabsf(v1)));
    code = mx::e8m0_code(amax);
    const float inv = mx::e8m0_inv_scale(code);
    uint32_t byte = mx::e2m1_code(v0 * inv) | (mx::e2m1_code(v1 * inv) << 4);
    byte |= (uint32_t)mx::dpp<mx::kDppQuadNext1>((int)byte) << 8;    // lane 4j: bytes of 4j..4j+3
    byte |= (uint32_t)mx::dpp<mx::kDppQuadNext2>((int)byte) << 16;
    bytes4 = byte;
}

}  // namespace am
