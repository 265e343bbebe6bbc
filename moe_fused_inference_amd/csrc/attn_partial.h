// attn_partial.h -- the chunk pass of decode attention over the FP8 (E4M3)
// KV cache, as a device function shared by attn_partial_kernel (attn.hip)
// and the decode layer launch that runs the next layer's chunk pass after
// its q|k|v projection (decode_layer.hip).  The q|k|v values come through a
// source type: plain loads of the projection rows, or, inside the layer
// launch, the (value, tag) words its projection workgroups publish.
//
// The byte codec is the reference's own (f32_to_e4m3 / e4m3_to_f32 at
// src/ext/mxfp4_decode.cu:355-364,437-455), see kv_codec.h.
#pragma once
#include "attn_merge.h"
#include "head_rope.h"
#include "kv_codec.h"
#include "mx_device.h"

namespace ap {

using am::kChunk;
using am::kD;
using am::kPart;
using kv::e4m3_ref_decode;

constexpr int kMaxFusedM = 16;   // tokens per call of the fused entry (the decode step's M)

// The fused entry's extra inputs: the fp32 q|k|v projection rows (M, (Hq +
// 2 Hkv) D), the q/k RMSNorm weights, RoPE theta and the KV byte codec; the
// cache is written through kvk_w / kvv_w.
struct QkvIn {
    const float* qkv;
    const uint16_t* qw;
    const uint16_t* kw;
    float eps, theta;
    int codec;
    uint8_t* kvk_w;
    uint8_t* kvv_w;
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// D (16 x 16 fp32) += A (16 x 32 bf16) B (32 x 16 bf16); lane l holds row /
// column l % 16 of A / B and 8 values of the reduction dimension, the same 8
// for A and B (which 8 is immaterial as long as both sides agree); D[4*(l/16)
// + i][l % 16] is element i of the lane's result.
__device__ __forceinline__ mx::v4f mfma_bf16(uint4 a, uint4 b, mx::v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
}

// A cache byte (the reference's codec) as bf16 bits: every value of the
// codec, 840 included, is a bf16 value, so this is exact.
__device__ __forceinline__ uint32_t kv_bf16(uint32_t b) { return __float_as_uint(e4m3_ref_decode(b)) >> 16; }
__device__ __forceinline__ uint32_t pack_bf16(uint32_t lo, uint32_t hi) { return lo | (hi << 16); }
// The same through a 256-entry LDS table of the codec's bf16 bits (lut[b]
// = kv_bf16(b), built once per workgroup): one LDS read per byte instead of
// the codec's ~12 instructions.
__device__ __forceinline__ uint32_t kv_lut(const uint16_t* lut, uint32_t b) { return lut[b & 0xFFu]; }
__device__ __forceinline__ uint4 kv8_bf16(const uint16_t* lut, uint2 w) {
    return make_uint4(pack_bf16(kv_lut(lut, w.x), kv_lut(lut, w.x >> 8)),
                      pack_bf16(kv_lut(lut, w.x >> 16), kv_lut(lut, w.x >> 24)),
                      pack_bf16(kv_lut(lut, w.y), kv_lut(lut, w.y >> 8)),
                      pack_bf16(kv_lut(lut, w.y >> 16), kv_lut(lut, w.y >> 24)));
}


// The chunk pass's LDS.
template <int RT, bool FUSED>
struct AttnLds {
    static constexpr int R = 16 * RT;
    alignas(16) uint16_t qs[R][kD + 8];          // 272-byte rows: conflict-free operand reads
    alignas(16) uint16_t phi[R][kChunk + 8];     // p, bf16 high part
    alignas(16) uint16_t plo[R][kChunk + 8];     // p - high, bf16
    float red[4][R];
    float rstat[2][R];
    uint16_t lut[256];
    alignas(16) uint8_t knew[FUSED ? kChunk : 1][kD];
    alignas(16) uint8_t vnew[FUSED ? kChunk : 1][kD];
    float2 rcs[FUSED ? kMaxFusedM : 1][64];
};

// q|k|v values by plain loads of the fp32 projection rows.
struct PlainQkv {
    static constexpr bool kWaits = false;
    const float* qkv;
    template <int QR, int NR>
    __device__ __forceinline__ bool fetch(const int64_t (&qo)[QR], const int64_t (&ko)[NR], float (&qa)[QR],
                                          float (&qb)[QR], float (&ka)[NR], float (&kb)[NR]) const {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < QR; ++i) {
            qa[i] = qkv[qo[i] + lane];
            qb[i] = qkv[qo[i] + lane + 64];
        }
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            ka[j] = qkv[ko[j] + lane];
            kb[j] = qkv[ko[j] + lane + 64];
        }
        return true;
    }
};

// Workgroup (64-position chunk, kv head g, MT consecutive tokens): R = 16*RT
// query rows, row r = (token m0 + r / G, head g*G + r % G), all sharing the
// chunk's K and V rows, which are loaded and decoded once.
//  1. loads first: K bytes in the MFMA operand layout (wave w: positions
//     16w..16w+15), V bytes likewise (wave w: columns 32w..32w+31, 8
//     positions a lane), q rows to LDS; the position only masks (rows past
//     max_pos are clamped), so the workgroup pays one memory latency;
//  2. S = Q K^T on MFMA (bf16 q, bf16-exact K, fp32 accumulation), the raw
//     scores to sc;
//  3. per row the chunk max, p = exp(x - max) and the sum (LDS across waves);
//  4. O = P V on MFMA with p split into bf16 high + low parts (the low part
//     carries p - high exactly enough that the product is fp32-accurate);
//  -> one record (max, sum, 128 column sums) per (token, head, chunk).
//
// FUSED: q and the step's new K / V rows come from the fp32 projections
// instead (the qk_rope_kv_kernel arithmetic, head_rope.h and kv_codec.h, so
// the bits are the same): each workgroup normalises and rotates the q rows
// of its heads into LDS, and a workgroup whose chunk holds positions of this
// step (dpos .. dpos+M-1) encodes those tokens' k / v rows of its kv head,
// uses them in place of the cache bytes, which are not written yet, and
// writes the rows of its own tokens to the cache.
//
// The workgroup is (chunk, g, token group mz); L is its LDS.  FUSED takes the
// projection values through `src`: src.fetch(qo, ko, qa, qb, ka, kb) fills
// qa[i] / qb[i] with elements lane / lane + 64 of the q|k|v row starting at
// element qo[i] (ka / kb likewise from ko[j]) and returns false if they could
// not be had (values then zero); QSRC::kWaits says the fetch waits for them
// to be produced (the RoPE tables are then built before it, not under it).
template <int G, int RT, bool FUSED, class QSRC>
__device__ __forceinline__ void attn_partial_body(AttnLds<RT, FUSED>& L, const QSRC& src, int chunk, int g, int mz,
                                                  const uint16_t* __restrict__ q,
                                                  const uint8_t* kvk,   // FUSED writes rows of it
                                                  const uint8_t* kvv, float* __restrict__ sc,
                                                  float* __restrict__ part, const int32_t* __restrict__ dpos, int M,
                                                  int Hq, int Hkv, int max_pos, int nchunk, float invsqrt,
                                                  const QkvIn& fz) {
    constexpr int R = 16 * RT;
    constexpr int MT = R / G;
    static_assert(R % G == 0 && MT >= 1, "rows hold whole tokens");
    const int m0 = mz * MT;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lq = lane >> 4;
    const int s0 = chunk * kChunk;
    const int rowmax = max_pos - 1 - s0;       // last in-bounds row of the chunk (s0 < max_pos)
    const int64_t rs = (int64_t)Hkv * kD;      // bytes per cache row
    auto& qs = L.qs;
    auto& phi = L.phi;
    auto& plo = L.plo;
    auto& red = L.red;
    auto& rstat = L.rstat;
    auto& lut = L.lut;
    lut[tid] = (uint16_t)kv_bf16((uint32_t)tid);   // 256 threads: one entry each
    // ---- 1. loads
    uint2 kraw[4];
    {
        const uint8_t* kr = kvk + (int64_t)(s0 + min(wave * 16 + l16, rowmax)) * rs + g * kD + lq * 8;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kraw[kt] = *reinterpret_cast<const uint2*>(kr + kt * 32);
    }
    uint32_t vraw[2][2][8];
    {
        const uint8_t* vc = kvv + g * kD + wave * 32 + l16;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    vraw[c][kt][t] = vc[(int64_t)(s0 + min(kt * 32 + lq * 8 + t, rowmax)) * rs + c * 16];
    }
    const int base = *dpos;
    // with a waiting q|k|v source: K / V as bf16 MFMA operands, decoded ahead
    uint4 kdec[QSRC::kWaits ? 4 : 1], vdec[QSRC::kWaits ? 2 : 1][2];
    auto decode_v = [&](int kt, int c) {
        const uint32_t* v = vraw[c][kt];
        return make_uint4(pack_bf16(kv_lut(lut, v[0]), kv_lut(lut, v[1])), pack_bf16(kv_lut(lut, v[2]), kv_lut(lut, v[3])),
                          pack_bf16(kv_lut(lut, v[4]), kv_lut(lut, v[5])), pack_bf16(kv_lut(lut, v[6]), kv_lut(lut, v[7])));
    };
    auto decode_all = [&]() {
        if constexpr (QSRC::kWaits) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) kdec[kt] = kv8_bf16(lut, kraw[kt]);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int c = 0; c < 2; ++c) vdec[kt][c] = decode_v(kt, c);
        }
    };
    if (!FUSED) {
        for (int i = tid; i < R * 16; i += 256) {
            const int r = i >> 4, c = i & 15;
            const int m = m0 + r / G;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (m < M) v = *reinterpret_cast<const uint4*>(q + ((int64_t)m * Hq + g * G + r % G) * kD + c * 8);
            *reinterpret_cast<uint4*>(&qs[r][c * 8]) = v;
        }
    }
    // FUSED: this step's k / v rows that fall in the chunk, [n_lo, n_hi)
    auto& knew = L.knew;
    auto& vnew = L.vnew;
    const int n_lo = max(base, s0), n_hi = min(min(base + M, s0 + kChunk), max_pos);
    if (FUSED) {
        const int nh = Hq + 2 * Hkv;
        // every projection value the wave needs is loaded first (one memory
        // round trip, under the K / V loads above): q rows r = wave + 4i,
        // and the tasks t = wave + 4j of the step's new rows in this chunk
        // (task t: row n_lo + t/2, its k for even t, its v for odd t)
        constexpr int QR = (R + 3) / 4;
        constexpr int NR = (2 * kMaxFusedM + 3) / 4;
        float qa[QR], qb[QR], ka[NR], kb[NR];
        const uint16_t wqa = fz.qw[lane], wqb = fz.qw[lane + 64], wka = fz.kw[lane], wkb = fz.kw[lane + 64];
        // (unconditional loads of clamped rows, unused values zeroed after:
        // a load inside a branch would be waited for before the branch joins)
        int64_t qo[QR], ko[NR];
#pragma unroll
        for (int i = 0; i < QR; ++i) {
            const int r = wave + 4 * i, m = m0 + r / G;
            qo[i] = ((int64_t)min(m, M - 1) * nh + g * G + r % G) * kD;
        }
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int t = wave + 4 * j, tok = min(max(n_lo + (t >> 1) - base, 0), M - 1);
            ko[j] = ((int64_t)tok * nh + (t & 1 ? Hq + Hkv : Hq) + g) * kD;
        }
        // RoPE cos / sin of every position the workgroup needs -- its own
        // tokens and the step's rows in its chunk -- once per (token, lane)
        // in LDS: a wave would otherwise evaluate them for each of its
        // tokens (pow, cos and sin cost hundreds of instructions)
        auto& rcs = L.rcs;
        auto rope_tables = [&]() {
            for (int jm = wave; jm < M; jm += 4) {   // token jm
                const bool own = jm >= m0 && jm < m0 + MT;
                const bool newrow = base + jm >= n_lo && base + jm < n_hi;
                if (own || newrow) rcs[jm][lane] = hr::rope_cs(fz.theta, lane, base + jm);
            }
        };
        if constexpr (QSRC::kWaits) {
            // the wait for q is long: decode the cache bytes to bf16 and build
            // the RoPE tables before it, off the critical path
            __syncthreads();   // lut
            decode_all();
            rope_tables();
        }
        src.template fetch<QR, NR>(qo, ko, qa, qb, ka, kb);
        if constexpr (!QSRC::kWaits) rope_tables();
#pragma unroll
        for (int i = 0; i < QR; ++i) {
            const bool ok = m0 + (wave + 4 * i) / G < M;
            qa[i] = ok ? qa[i] : 0.0f;
            qb[i] = ok ? qb[i] : 0.0f;
        }
        __syncthreads();
        // q: RMSNorm + RoPE at the token's position, bf16 into LDS; rows of
        // tokens past M are zeros.  No branch per row, so the rows'
        // reductions can interleave.  With G % 4 == 0 a wave's rows of token
        // m0 + tt are i = tt*G/4 .. (tt+1)*G/4 - 1 (r / G = tt), so one
        // uniform branch per token skips the tokens past M.
        if constexpr (G % 4 == 0) {
            constexpr int RPT = G / 4;
#pragma unroll
            for (int tt = 0; tt < MT; ++tt) {
                if (m0 + tt < M) {
#pragma unroll
                    for (int ii = 0; ii < RPT; ++ii) {
                        const int i = tt * RPT + ii, r = wave + 4 * i;
                        uint16_t ba, bb;
                        hr::norm_rope(qa[i], qb[i], mx::bf16_to_f32(wqa), mx::bf16_to_f32(wqb), fz.eps,
                                      rcs[m0 + tt][lane], ba, bb);
                        qs[r][lane] = ba;
                        qs[r][lane + 64] = bb;
                    }
                } else {
#pragma unroll
                    for (int ii = 0; ii < RPT; ++ii) {
                        const int r = wave + 4 * (tt * RPT + ii);
                        qs[r][lane] = qs[r][lane + 64] = 0;
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < QR; ++i) {
                const int r = wave + 4 * i, m = m0 + r / G;
                uint16_t ba, bb;
                hr::norm_rope(qa[i], qb[i], mx::bf16_to_f32(wqa), mx::bf16_to_f32(wqb), fz.eps,
                              rcs[min(m, M - 1)][lane], ba, bb);
                qs[r][lane] = m < M ? ba : (uint16_t)0;
                qs[r][lane + 64] = m < M ? bb : (uint16_t)0;
            }
        }
        // the new rows: k (RMSNorm + RoPE) and bf16(v) as cache bytes, to
        // LDS, and the rows of this workgroup's tokens to the cache
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int t = wave + 4 * j, p = n_lo + (t >> 1);
            if (p >= n_hi) break;
            const int m = p - base;
            float e0, e1;   // the values to encode
            if (t & 1) {    // v: bf16(v)
                e0 = mx::bf16_to_f32(mx::f32_to_bf16_rne(ka[j]));
                e1 = mx::bf16_to_f32(mx::f32_to_bf16_rne(kb[j]));
            } else {        // k: RMSNorm + RoPE at its position
                uint16_t ba, bb;
                hr::norm_rope(ka[j], kb[j], mx::bf16_to_f32(wka), mx::bf16_to_f32(wkb), fz.eps, rcs[m][lane], ba, bb);
                e0 = mx::bf16_to_f32(ba);
                e1 = mx::bf16_to_f32(bb);
            }
            const uint8_t b0 = (uint8_t)kv::e4m3_encode(e0, fz.codec);
            const uint8_t b1 = (uint8_t)kv::e4m3_encode(e1, fz.codec);
            uint8_t (*dst)[kD] = t & 1 ? vnew : knew;
            dst[p - s0][lane] = b0;
            dst[p - s0][lane + 64] = b1;
            if (m >= m0 && m < m0 + MT) {
                uint8_t* c = (t & 1 ? fz.kvv_w : fz.kvk_w) + ((int64_t)p * Hkv + g) * kD;
                c[lane] = b0;
                c[lane + 64] = b1;
            }
        }
    }
    // tokens m0..m0+MT-1 sit at positions base + m; those inside [0, max_pos) count
    const int mv_lo = max(m0, -base);
    const int mv_hi = min(min(M, m0 + MT) - 1, max_pos - 1 - base);
    if (mv_hi < mv_lo || s0 > base + mv_hi) return;   // uniform: no token of this workgroup reaches the chunk
    __syncthreads();
    if (FUSED && n_lo < n_hi) {
        // the step's rows in place of the cache bytes loaded above
        const int kr = s0 + wave * 16 + l16;
        if (kr >= n_lo && kr < n_hi) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                kraw[kt] = *reinterpret_cast<const uint2*>(&knew[kr - s0][kt * 32 + lq * 8]);
                if constexpr (QSRC::kWaits) kdec[kt] = kv8_bf16(lut, kraw[kt]);   // decoded ahead: again
            }
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                bool changed = false;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int vr = s0 + kt * 32 + lq * 8 + t;
                    if (vr >= n_lo && vr < n_hi) {
                        vraw[c][kt][t] = vnew[vr - s0][wave * 32 + l16 + c * 16];
                        changed = true;
                    }
                }
                if constexpr (QSRC::kWaits)
                    if (changed) vdec[kt][c] = decode_v(kt, c);
            }
    }
    // ---- 2. scores, wave = positions 16*wave + l16
    mx::v4f sacc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) sacc[rt] = mx::v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
        uint4 kb;
        if constexpr (QSRC::kWaits) kb = kdec[kt];
        else kb = kv8_bf16(lut, kraw[kt]);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            sacc[rt] = mfma_bf16(*reinterpret_cast<const uint4*>(&qs[rt * 16 + l16][kt * 32 + lq * 8]), kb, sacc[rt]);
    }
    // ---- 3. softmax statistics
    const int s = s0 + wave * 16 + l16;
    float x[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = rt * 16 + 4 * lq + i;
            const int m = m0 + r / G;
            const bool ok = m >= mv_lo && m <= mv_hi && s <= base + m;
            if (ok && sc) sc[((int64_t)m * Hq + g * G + r % G) * max_pos + s] = sacc[rt][i];
            x[rt][i] = ok ? sacc[rt][i] * invsqrt : -INFINITY;
            const float mxv = mx::row16_reduce<true>(x[rt][i]);
            if (l16 == 0) red[wave][r] = mxv;
        }
    __syncthreads();
    if (tid < R) rstat[0][tid] = fmaxf(fmaxf(red[0][tid], red[1][tid]), fmaxf(red[2][tid], red[3][tid]));
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = rt * 16 + 4 * lq + i;
            const float mr = rstat[0][r];
            const float p = mr == -INFINITY ? 0.0f : expf(x[rt][i] - mr);   // exp(-inf) = 0 for masked positions
            const uint16_t hi = mx::f32_to_bf16_rne(p);
            phi[r][wave * 16 + l16] = hi;
            plo[r][wave * 16 + l16] = mx::f32_to_bf16_rne(p - mx::bf16_to_f32(hi));
            const float sum = mx::row16_reduce<false>(p);
            if (l16 == 0) red[wave][r] = sum;
        }
    __syncthreads();
    if (tid < R) rstat[1][tid] = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
    // ---- 4. O = P V, wave = columns 32*wave + 16c + l16
    mx::v4f oacc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) oacc[rt][0] = oacc[rt][1] = mx::v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        uint4 vb[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            if constexpr (QSRC::kWaits) vb[c] = vdec[kt][c];
            else vb[c] = decode_v(kt, c);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint4 ah = *reinterpret_cast<const uint4*>(&phi[rt * 16 + l16][kt * 32 + lq * 8]);
            const uint4 al = *reinterpret_cast<const uint4*>(&plo[rt * 16 + l16][kt * 32 + lq * 8]);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                oacc[rt][c] = mfma_bf16(ah, vb[c], oacc[rt][c]);
                oacc[rt][c] = mfma_bf16(al, vb[c], oacc[rt][c]);
            }
        }
    }
    __syncthreads();                           // rstat[1]
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = rt * 16 + 4 * lq + i;
            const int m = m0 + r / G;
            if (m < mv_lo || m > mv_hi || s0 > base + m) continue;   // no record: the merge reads chunks up to the token's position
            float* rec = part + (((int64_t)m * Hq + g * G + r % G) * nchunk + chunk) * kPart;
#pragma unroll
            for (int c = 0; c < 2; ++c) rec[4 + wave * 32 + c * 16 + l16] = oacc[rt][c][i];
            if (wave == 0 && l16 == 0) {
                rec[0] = rstat[0][r];
                rec[1] = rstat[1][r];
            }
        }
}

}  // namespace ap
