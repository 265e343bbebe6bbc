// decode_layer.hip -- one-launch decode MoE layer for gfx950 (batch 1).
//
// Replaces, for one token, the reference's per-layer sequence
//   prequant -> moe_gateup -> moe_down -> moe_combine -> x + moe.bfloat16()
// (runtime/model_runner_v2.py:185-208; kernels src/ext/mxfp4_decode.cu:24-50,
// 177-299) with a single kernel, on un-quantized bf16 activations: the
// dequant-to-BF16 path of runtime/model_runner.py:128-131 computed in fp32,
// which is the north-star tolerance oracle.
//
// HBM-bound GEMV (20.05 MB of packed weights per layer at top-8, H=2048,
// Mi=768), so the design goal is to have every weight byte of the layer in
// flight from the first microsecond:
//
//   workgroups [0, nA)      gate/up: slot s, 32 intermediate rows j0..j0+31 of
//                           both gate and up (64 rows x K=H), K split over the
//                           4 waves; computes h = silu(g)*u in fp32 and
//                           publishes it, then increments an arrival counter.
//   workgroups [nA, nA+nB)  down + combine: 16 output columns for all E slots.
//                           They load their down weights first, then wait on
//                           the arrival counter (bounded), then run 2 slots per
//                           wave and combine sum_e w_e*y_e in-workgroup, adding
//                           the bf16 residual as the reference does.
//
// Synchronisation.  Workgroups are dispatched in index order, so every
// gate/up workgroup is resident or finished before any down workgroup waits:
// the wait cannot deadlock.  It is still bounded (kSpinLimit polls); on expiry
// the kernel sets an error flag, skips its work and exits normally.
//   * Each gate/up workgroup publishes its 32 values of h with agent-scope
//     atomic stores (write-through to the device coherence point), drains its
//     store counter (s_waitcnt vmcnt(0)), then bumps the arrival counter of
//     its slot -- one counter per slot, each in its own cache line, so the
//     Mi/32 increments per slot do not all serialise on one address.  (A
//     release/acquire fence pair would instead write back and invalidate a
//     whole L2 per workgroup.)
//   * Counters only ever grow.  Down workgroup b keeps, in the workspace, the
//     count it expects for each slot ("memo"); it waits until every slot's
//     counter reaches memo + Mi/32, reads h with agent-scope loads and stores
//     the new memo.  All counters and memos advance by the same amount per
//     launch, so no reset and no departure counter are needed between
//     launches or graph replays.  A workspace is tied to one H (the set of
//     down workgroups); mxfp4_decode_layer_reset zeroes it.
//   * Within one launch every h line is written before any reader touches
//     it, and each launch starts with the dispatch-level cache invalidation,
//     so no reader can hold a stale copy.
//
// Registers are kept under 128 VGPRs (h is staged through LDS, the down
// K-step count is a template bound) so that every workgroup of a layer is
// resident from the start and all weight loads are in flight at once.
//
// Activations on the MFMA: there is no bf16 x FP4 MFMA, so the bf16 x (and the
// fp32 h) is split into three E4M3 terms hi + mid + lo, each with its own E8M0
// 32-block scale, that sum back to the value to about 12 significant bits
// (exactly, for bf16 x).  The three terms are rows 0..2 of the 16-row A
// operand of v_mfma_scale_f32_16x16x128_f8f6f4 (A = E4M3, B = E2M1), so one
// MFMA yields all three partial products and y = D[0] + D[1] + D[2]; the other
// 13 rows are zero and cost nothing in an HBM-bound kernel.
#include "mx_device.h"
#include "mx_host.h"

namespace {

constexpr int kSpinLimit = 1 << 22;   // polls of the arrival counters (~0.2 s)
constexpr int kTerms = 3;             // E4M3 terms per activation value
constexpr int kMaxE = 8;
// workspace layout (bytes)
constexpr int kCtrOff = 0;            // int32 counter of slot s at kCtrOff + 128*s
constexpr int kErrOff = 1024;         // int32 error flag
constexpr int kMemoOff = 2048;        // int32 memo[H/16][8]
constexpr int kHOff = 8192;           // h terms, then h scale codes

struct LayerArgs {
    const uint16_t* x;        // (H) bf16
    const uint8_t* gate_wp;   // expert e at + e*wp_stride_gu: (Mi, H/2)
    const uint8_t* gate_ws;   //                               (Mi, H/32)
    const uint8_t* up_wp;
    const uint8_t* up_ws;
    const uint8_t* down_wp;   // (H, Mi/2)
    const uint8_t* down_ws;   // (H, Mi/32)
    int64_t wp_stride_gu, ws_stride_gu;   // bytes between experts (gate/up)
    int64_t wp_stride_dn, ws_stride_dn;   // bytes between experts (down)
    const int32_t* ids_dev;   // (E) expert ids in device memory, or null
    const float* w_dev;       // (E) combine weights in device memory, or null
    int32_t ids[kMaxE];       // by-value ids when ids_dev is null
    float w[kMaxE];           // by-value weights when w_dev is null
    int E, H, Mi;
    float* out;               // (H) fp32 moe output
    uint16_t* resid;          // (H) bf16 x + bf16(out), or null
    uint8_t* ws;              // workspace base
    uint8_t* hs8;             // (E, kTerms, Mi) E4M3 terms of h
    uint32_t* hsc;            // (E, Mi/32) scale codes of terms 0..2 in bytes 0..2
};

// E8M0 code of the smallest 2^e with amax <= 448*2^e (E4M3 range), e in
// [-127, 127]; zero blocks get 127.
__device__ __forceinline__ uint32_t e4m3_block_code(float amax) {
    if (!(amax > 0.0f)) return 127u;
    uint32_t bits = __float_as_uint(amax);
    int ex = (int)(bits >> 23);
    uint32_t frac = bits & 0x7FFFFFu;
    int x;
    if (ex == 0) {
        int p = 31 - __clz((int)frac);
        x = p - 149;
        frac = (frac << (23 - p)) & 0x7FFFFFu;
    } else {
        x = ex - 127;
    }
    int e = (frac <= 0x600000u) ? x - 8 : x - 7;  // (1+f) <= 1.75 -> 448 fits
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
    return (uint32_t)(e + 127);
}

__device__ __forceinline__ float e8m0_value(uint32_t code) {
    return code > 0u ? __uint_as_float(code << 23) : __uint_as_float(0x00400000u);
}

// Splits 8 consecutive values of a 32-block (4 lanes per block, lane quad
// aligned) into kTerms E4M3 terms: word8[t] receives the 8 E4M3 bytes of term
// t and codes (byte t) the term's E8M0 scale code.  Each term is the E4M3
// rounding of what the previous terms left over, so the terms sum to the value
// up to the last term's rounding (exact for bf16 inputs).
__device__ __forceinline__ void split8(float v[8], uint64_t word8[kTerms], uint32_t& codes) {
    codes = 0;
#pragma unroll
    for (int t = 0; t < kTerms; ++t) {
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) am = fmaxf(am, __builtin_fabsf(v[i]));
        am = fmaxf(am, __shfl_xor(am, 1));
        am = fmaxf(am, __shfl_xor(am, 2));
        const uint32_t code = e4m3_block_code(am);
        const float sc = e8m0_value(code);
        uint32_t word[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            mx::v2s p = {0, 0};
            p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, v[4 * h + 0], v[4 * h + 1], sc, false);
            p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, v[4 * h + 2], v[4 * h + 3], sc, true);
            word[h] = ((uint32_t)(uint16_t)p[0]) | ((uint32_t)(uint16_t)p[1] << 16);
            typedef float v2f __attribute__((ext_vector_type(2)));
            const v2f d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word[h], sc, false);
            const v2f d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word[h], sc, true);
            v[4 * h + 0] -= d0[0];
            v[4 * h + 1] -= d0[1];
            v[4 * h + 2] -= d1[0];
            v[4 * h + 3] -= d1[1];
        }
        word8[t] = (uint64_t)word[0] | ((uint64_t)word[1] << 32);
        codes |= code << (8 * t);
    }
}

// Expert id / weight of slot s from the by-value arrays with a uniform index
// (scalar selects, no indexed load of the kernel-argument block).
__device__ __forceinline__ int pick_id(const LayerArgs& a, int s) {
    int e = a.ids[0];
#pragma unroll
    for (int k = 1; k < kMaxE; ++k) e = (s == k) ? a.ids[k] : e;
    return e;
}
__device__ __forceinline__ float pick_w(const LayerArgs& a, int s) {
    float w = a.w[0];
#pragma unroll
    for (int k = 1; k < kMaxE; ++k) w = (s == k) ? a.w[k] : w;
    return w;
}

__device__ __forceinline__ void drain_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Unconditional load from an always-valid (clamped) address, value selected
// afterwards: keeps every load of a phase in one basic block so the compiler
// can wait for exactly the loads a computation needs.
template <typename T>
__device__ __forceinline__ T ld_sel(const T* p, bool ok, T zero) {
    const T v = *p;
    return ok ? v : zero;
}

// FP8-A operand of one MFMA K-step for lane (r = term row, g) when B lane
// group gb holds 32-block phys(gb) of this step: bytes 0..15 <- logical K
// 16g..16g+15 (B group g/2, elements 16*(g%2)..), bytes 16..31 <- logical K
// 64+16g.. (B group 2+g/2).
__device__ __forceinline__ mx::v8i fp8_operand(const uint8_t* row8, int blk_lo, int blk_hi, int g) {
    const uint4 lo = *reinterpret_cast<const uint4*>(row8 + blk_lo * 32 + 16 * (g & 1));
    const uint4 hi = *reinterpret_cast<const uint4*>(row8 + blk_hi * 32 + 16 * (g & 1));
    mx::v8i a = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    return a;
}

union Smem {
    struct {                                       // gate/up workgroups
        uint8_t x8[kTerms][2048];                  // E4M3 terms of x (H <= 2048)
        uint8_t xsc[kTerms][64];
        float red[4][4][16];
        float h[2][32];
    } a;
    struct {                                       // down workgroups
        uint8_t h8[kMaxE * kTerms * 1024];         // E4M3 terms of h (Mi <= 1024)
        uint32_t hsc[kMaxE * 32];
        float red[4][16];
        int abort;
    } b;
};

template <bool DEV_IDS, int MS>
__global__ __launch_bounds__(256) void decode_layer_kernel(LayerArgs a) {
    __shared__ __align__(16) Smem sm;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const int nblk_mi = a.Mi >> 5;
    const int nA = a.E * nblk_mi;
    const int bid = blockIdx.x;
    int* ctr = reinterpret_cast<int*>(a.ws + kCtrOff);

    if (bid < nA) {
        // ================================================= gate / up
        const int s = bid % a.E;
        const int jb = bid / a.E;
        const int j0 = jb * 32;
        const int H = a.H;
        const int hb = H >> 5;                  // 32-blocks per row (64)
        const int bpw = hb >> 2;                // blocks per wave (16)
        const int sa = bpw >> 2;                // K-steps per wave (H/512, <= 4)

        // x first: its value is needed before the MFMAs, the weights only by them
        const int k0 = threadIdx.x * 8;
        uint4 xq = make_uint4(0, 0, 0, 0);
        if (k0 < H) xq = *reinterpret_cast<const uint4*>(a.x + k0);

        const int e = DEV_IDS ? __builtin_amdgcn_readfirstlane(a.ids_dev[s]) : pick_id(a, s);
        const uint8_t* gw = a.gate_wp + (int64_t)e * a.wp_stride_gu;
        const uint8_t* gs = a.gate_ws + (int64_t)e * a.ws_stride_gu;
        const uint8_t* uw = a.up_wp + (int64_t)e * a.wp_stride_gu;
        const uint8_t* us = a.up_ws + (int64_t)e * a.ws_stride_gu;

        // weights: 4 row groups (gate lo/hi, up lo/hi) x sa K-steps; lane
        // group g owns blocks bpw*wave + sa*g .. +sa-1 of its row (contiguous)
        uint4 bq[4][4];
        uint32_t bsc4[4];
        const int blk0 = bpw * wave + sa * g;
#pragma unroll
        for (int G = 0; G < 4; ++G) {
            const int row = j0 + 16 * (G & 1) + r;
            const uint8_t* wrow = ((G < 2) ? gw : uw) + (int64_t)row * (H >> 1);
            const uint8_t* srow = ((G < 2) ? gs : us) + (int64_t)row * hb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int blk = min(blk0 + i, hb - 1);
                bq[G][i] = ld_sel(reinterpret_cast<const uint4*>(wrow + blk * 16), i < sa, make_uint4(0, 0, 0, 0));
            }
            // scale bytes blk0..blk0+sa-1 (sa <= 4) from the two dwords around
            // them; bytes past sa belong to zero data and are ignored
            const int d0 = blk0 & ~3;
            const uint32_t lo = *reinterpret_cast<const uint32_t*>(srow + d0);
            const uint32_t hi = *reinterpret_cast<const uint32_t*>(srow + min(d0 + 4, hb - 4));
            bsc4[G] = (uint32_t)((((uint64_t)hi << 32) | lo) >> (8 * (blk0 & 3)));
        }

        // x -> three E4M3 terms in LDS (whole row; 8 values per thread)
        if (k0 < H) {
            float v[8];
            const uint32_t w4[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = mx::bf16_to_f32((uint16_t)(w4[i] & 0xFFFFu));
                v[2 * i + 1] = mx::bf16_to_f32((uint16_t)(w4[i] >> 16));
            }
            uint64_t w8[kTerms];
            uint32_t codes;
            split8(v, w8, codes);
#pragma unroll
            for (int t = 0; t < kTerms; ++t) {
                *reinterpret_cast<uint64_t*>(&sm.a.x8[t][k0]) = w8[t];
                if ((threadIdx.x & 3) == 0) sm.a.xsc[t][k0 >> 5] = (uint8_t)(codes >> (8 * t));
            }
        }
        __syncthreads();

        // MFMA: step i covers blocks {bpw*wave + sa*gb + i : gb = 0..3}
        mx::v4f acc[4];
#pragma unroll
        for (int G = 0; G < 4; ++G) acc[G] = (mx::v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i >= sa) break;
            mx::v8i av = {0, 0, 0, 0, 0, 0, 0, 0};
            uint32_t asc = 127u;
            if (r < kTerms) {
                const int base = bpw * wave + i;
                av = fp8_operand(sm.a.x8[r], base + sa * (g >> 1), base + sa * (2 + (g >> 1)), g);
                asc = sm.a.xsc[r][base + sa * g];
            }
#pragma unroll
            for (int G = 0; G < 4; ++G)
                acc[G] = mx::mfma16_fp8a_fp4b(av, bq[G][i], acc[G], asc, (bsc4[G] >> (8 * i)) & 0xFFu);
        }
        // rows 0..2 of D (the three terms) are elements 0..2 of lanes 0..15
        if (lane < 16) {
#pragma unroll
            for (int G = 0; G < 4; ++G) sm.a.red[wave][G][lane] = acc[G][0] + acc[G][1] + acc[G][2];
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            const int G = threadIdx.x >> 4;   // 0,1 gate halves; 2,3 up halves
            const int n = threadIdx.x & 15;
            sm.a.h[G >> 1][16 * (G & 1) + n] =
                sm.a.red[0][G][n] + sm.a.red[1][G][n] + sm.a.red[2][G][n] + sm.a.red[3][G][n];
        }
        __syncthreads();
        // h = silu(g) * u for the 32 rows, split into E4M3 terms, published
        // with agent-scope stores; then the slot's arrival counter
        if (threadIdx.x < 4) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int j = threadIdx.x * 8 + i;
                v[i] = mx::silu_mul(sm.a.h[0][j], sm.a.h[1][j]);
            }
            uint64_t w8[kTerms];
            uint32_t codes;
            split8(v, w8, codes);
#pragma unroll
            for (int t = 0; t < kTerms; ++t) {
                uint64_t* dst = reinterpret_cast<uint64_t*>(a.hs8 + ((int64_t)s * kTerms + t) * a.Mi + j0 + threadIdx.x * 8);
                __hip_atomic_store(dst, w8[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (threadIdx.x == 0)
                __hip_atomic_store(a.hsc + (int64_t)s * nblk_mi + jb, codes, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            drain_stores();
            if (threadIdx.x == 0)
                __hip_atomic_fetch_add(ctr + 32 * s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    // ===================================================== down + combine
    const int cb = bid - nA;
    const int c0 = cb * 16;
    const int Mi = a.Mi;
    const int kb = Mi >> 5;          // 32-blocks per down row (24)
    const int steps = (kb + 3) >> 2; // MFMA K-steps (6), <= MS
    // wave handles slots 2*wave, 2*wave+1; lane group g owns blocks
    // g*steps .. g*steps+steps-1 of its row
    int slot[2], eid[2];
    float wgt[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        slot[q] = 2 * wave + q;
        const int sl = slot[q] < a.E ? slot[q] : 0;
        eid[q] = DEV_IDS ? __builtin_amdgcn_readfirstlane(a.ids_dev[sl]) : pick_id(a, sl);
        wgt[q] = DEV_IDS ? a.w_dev[sl] : pick_w(a, sl);
    }
    uint4 bq[2][MS];
    uint32_t bsw[2][3];   // dwords holding the scale bytes of blocks g*steps..
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const bool live = slot[q] < a.E;
        const uint8_t* wrow = a.down_wp + (int64_t)eid[q] * a.wp_stride_dn + (int64_t)(c0 + r) * (Mi >> 1);
        const uint8_t* srow = a.down_ws + (int64_t)eid[q] * a.ws_stride_dn + (int64_t)(c0 + r) * kb;
#pragma unroll
        for (int i = 0; i < MS; ++i) {
            const int blk = g * steps + i;
            bq[q][i] = ld_sel(reinterpret_cast<const uint4*>(wrow + min(blk, kb - 1) * 16),
                              live && i < steps && blk < kb, make_uint4(0, 0, 0, 0));
        }
        const int sb0 = (g * steps) & ~3;  // blocks [g*steps, +steps) lie in 12 bytes from here
        if ((kb & 3) == 0) {
#pragma unroll
            for (int d = 0; d < 3; ++d)  // raw dwords; blocks past the row are masked by zero data
                bsw[q][d] = *reinterpret_cast<const uint32_t*>(srow + min(sb0 + 4 * d, kb - 4));
        } else {  // rows not a dword multiple: byte loads, never past the row
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                uint32_t v = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int off = sb0 + 4 * d + b;
                    v |= ((live && off < kb) ? (uint32_t)srow[off] : 127u) << (8 * b);
                }
                bsw[q][d] = v;
            }
        }
    }

    // wait until every slot's counter reaches this workgroup's memo + Mi/32
    int* memo = reinterpret_cast<int*>(a.ws + kMemoOff) + cb * kMaxE;
    if (wave == 0) {
        const bool mine = lane < a.E;
        const int target = (mine ? memo[lane] : 0) + nblk_mi;
        int spins = 0;
        bool ok = true;
        while (true) {
            const int c = mine ? __hip_atomic_load(ctr + 32 * lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : target;
            if (__ballot(c - target < 0) == 0ull) break;
            __builtin_amdgcn_s_sleep(2);
            if (++spins >= kSpinLimit) {
                ok = false;
                break;
            }
        }
        if (mine) memo[lane] = target;
        if (lane == 0) {
            if (!ok) __hip_atomic_store(reinterpret_cast<int*>(a.ws + kErrOff), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sm.b.abort = ok ? 0 : 1;
        }
    }
    __syncthreads();
    const bool abort = sm.b.abort != 0;

    // stage h (all slots, agent-scope loads) in LDS
    const int hbytes = a.E * kTerms * Mi;       // multiple of 96
    if (!abort) {
        uint64_t tmp[12];
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const int off = (threadIdx.x + 256 * k) * 8;
            tmp[k] = __hip_atomic_load(reinterpret_cast<const uint64_t*>(a.hs8 + min(off, hbytes - 8)),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const uint32_t hs = threadIdx.x < a.E * kb
                                ? __hip_atomic_load(a.hsc + threadIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : 0u;
#pragma unroll
        for (int k = 0; k < 12; ++k) {
            const int off = (threadIdx.x + 256 * k) * 8;
            if (off < hbytes) *reinterpret_cast<uint64_t*>(sm.b.h8 + off) = tmp[k];
        }
        if (threadIdx.x < a.E * kb) sm.b.hsc[threadIdx.x] = hs;
    }
    __syncthreads();

    float part = 0.0f;  // this lane's (lane < 16) partial combine over its slots
    if (!abort) {
        const int sb0 = (g * steps) & ~3;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (slot[q] >= a.E) continue;
            const uint8_t* h8 = sm.b.h8 + (slot[q] * kTerms + (r < kTerms ? r : 0)) * Mi;
            const uint32_t* hsq = sm.b.hsc + slot[q] * kb;
            mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < MS; ++i) {
                if (i >= steps) break;
                // step i: B lane group gb holds block gb*steps + i
                const int blo = (g >> 1) * steps + i;
                const int bhi = (2 + (g >> 1)) * steps + i;
                const int bown = g * steps + i;
                mx::v8i av = {0, 0, 0, 0, 0, 0, 0, 0};
                uint32_t asc = 127u;
                if (r < kTerms) {
                    const uint4 lo = blo < kb ? *reinterpret_cast<const uint4*>(h8 + blo * 32 + 16 * (g & 1))
                                              : make_uint4(0, 0, 0, 0);
                    const uint4 hi = bhi < kb ? *reinterpret_cast<const uint4*>(h8 + bhi * 32 + 16 * (g & 1))
                                              : make_uint4(0, 0, 0, 0);
                    av = (mx::v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
                    asc = bown < kb ? (hsq[bown] >> (8 * r)) & 0xFFu : 127u;
                }
                // weight scale byte of block g*steps+i from the aligned dwords
                const int bi = g * steps + i - sb0;           // 0..10
                const uint32_t wd = bi < 4 ? bsw[q][0] : (bi < 8 ? bsw[q][1] : bsw[q][2]);
                acc = mx::mfma16_fp8a_fp4b(av, bq[q][i], acc, asc, (wd >> (8 * (bi & 3))) & 0xFFu);
            }
            part = fmaf(wgt[q], acc[0] + acc[1] + acc[2], part);
        }
    }
    if (lane < 16) sm.b.red[wave][lane] = part;
    __syncthreads();
    if (!abort && threadIdx.x < 16) {
        const int c = c0 + threadIdx.x;
        const float y = sm.b.red[0][threadIdx.x] + sm.b.red[1][threadIdx.x] + sm.b.red[2][threadIdx.x] +
                        sm.b.red[3][threadIdx.x];
        a.out[c] = y;
        if (a.resid) {
            // runtime/model_runner_v2.py:208: x = x + moe.bfloat16() in bf16
            const float yb = mx::bf16_to_f32(mx::f32_to_bf16_rne(y));
            a.resid[c] = mx::f32_to_bf16_rne(mx::bf16_to_f32(a.x[c]) + yb);
        }
    }
}

__global__ void reset_workspace_kernel(int* ws, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) ws[i] = 0;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

extern "C" size_t mxfp4_decode_layer_workspace_size(int E, int Mi) {
    if (E <= 0 || Mi <= 0) return 0;
    return kHOff + align256((size_t)E * kTerms * Mi) + align256((size_t)E * (Mi / 32) * 4);
}

extern "C" int mxfp4_decode_layer_reset(void* workspace, void* stream) {
    MXH_REQUIRE(workspace, "decode_layer_reset: null workspace");
    hipLaunchKernelGGL(reset_workspace_kernel, dim3(1), dim3(256), 0, mxh::as_stream(stream),
                       static_cast<int*>(workspace), kHOff / 4);
    return mxh::launch_status("decode_layer_reset");
}

extern "C" int mxfp4_decode_layer_status(const void* workspace, int* error_flag) {
    MXH_REQUIRE(workspace && error_flag, "decode_layer_status: null pointer");
    int host = 0;
    hipError_t e = hipMemcpy(&host, static_cast<const uint8_t*>(workspace) + kErrOff, sizeof host,
                             hipMemcpyDeviceToHost);
    MXH_REQUIRE(e == hipSuccess, "decode_layer_status: %s", hipGetErrorString(e));
    *error_flag = host;
    return MXFP4_OK;
}

extern "C" int mxfp4_moe_decode_layer(const void* x, const int32_t* ids_host, const float* w_host,
                                      const int32_t* ids_dev, const float* w_dev,
                                      const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                                      const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws,
                                      int n_experts, int E, int H, int Mi, float* out, void* resid_out,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(x && gate_wp && gate_ws && up_wp && up_ws && down_wp && down_ws && out && workspace,
                "moe_decode_layer: null pointer");
    MXH_REQUIRE(E >= 1 && E <= kMaxE, "moe_decode_layer: E=%d must be in [1, 8]", E);
    MXH_REQUIRE(H % 512 == 0 && H >= 512 && H <= 2048, "moe_decode_layer: H=%d must be a multiple of 512 in [512, 2048]", H);
    MXH_REQUIRE(Mi % 32 == 0 && Mi >= 32 && Mi <= 1024, "moe_decode_layer: Mi=%d must be a multiple of 32 in [32, 1024]", Mi);
    MXH_REQUIRE((ids_dev != nullptr) == (w_dev != nullptr), "moe_decode_layer: give ids and weights both on device or both on host");
    MXH_REQUIRE(ids_dev || (ids_host && w_host), "moe_decode_layer: missing routing");
    MXH_REQUIRE(workspace_bytes >= mxfp4_decode_layer_workspace_size(E, Mi), "moe_decode_layer: workspace too small");
    MXH_REQUIRE(((uintptr_t)workspace & 255) == 0, "moe_decode_layer: workspace must be 256-byte aligned");
    MXH_REQUIRE(((uintptr_t)x & 15) == 0, "moe_decode_layer: x must be 16-byte aligned");
    LayerArgs a{};
    a.x = static_cast<const uint16_t*>(x);
    a.gate_wp = gate_wp;
    a.gate_ws = gate_ws;
    a.up_wp = up_wp;
    a.up_ws = up_ws;
    a.down_wp = down_wp;
    a.down_ws = down_ws;
    a.wp_stride_gu = (int64_t)Mi * (H / 2);
    a.ws_stride_gu = (int64_t)Mi * (H / 32);
    a.wp_stride_dn = (int64_t)H * (Mi / 2);
    a.ws_stride_dn = (int64_t)H * (Mi / 32);
    a.ids_dev = ids_dev;
    a.w_dev = w_dev;
    if (!ids_dev) {
        for (int s = 0; s < E; ++s) {
            MXH_REQUIRE(ids_host[s] >= 0 && ids_host[s] < n_experts, "moe_decode_layer: expert id %d out of range", ids_host[s]);
            a.ids[s] = ids_host[s];
            a.w[s] = w_host[s];
        }
    }
    a.E = E;
    a.H = H;
    a.Mi = Mi;
    a.out = out;
    a.resid = static_cast<uint16_t*>(resid_out);
    a.ws = static_cast<uint8_t*>(workspace);
    a.hs8 = a.ws + kHOff;
    a.hsc = reinterpret_cast<uint32_t*>(a.hs8 + align256((size_t)E * kTerms * Mi));
    const int nA = E * (Mi / 32);
    const int nB = H / 16;
    const int steps = (Mi / 32 + 3) / 4;
    hipStream_t st = mxh::as_stream(stream);
    if (steps <= 6) {
        if (ids_dev) hipLaunchKernelGGL((decode_layer_kernel<true, 6>), dim3(nA + nB), dim3(256), 0, st, a);
        else hipLaunchKernelGGL((decode_layer_kernel<false, 6>), dim3(nA + nB), dim3(256), 0, st, a);
    } else {
        if (ids_dev) hipLaunchKernelGGL((decode_layer_kernel<true, 8>), dim3(nA + nB), dim3(256), 0, st, a);
        else hipLaunchKernelGGL((decode_layer_kernel<false, 8>), dim3(nA + nB), dim3(256), 0, st, a);
    }
    return mxh::launch_status("moe_decode_layer");
}
