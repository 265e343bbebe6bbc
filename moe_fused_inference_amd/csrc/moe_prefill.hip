// moe_prefill.hip -- grouped MoE for prefill / batched tokens on gfx950.
//
// Replaces the per-expert Python loop of ModelRunnerV2.moe_compute
// (runtime/model_runner_v2.py:108-122):
//     for e in experts:
//         idx, slots = torch.where(topi == e)
//         g = forward(h[idx], gate_e); u = forward(h[idx], up_e)    # x -> half -> MXFP4
//         y = forward(silu(g) * u, down_e).to(bf16)                 # fp32 h -> half -> MXFP4
//         out.index_add_(0, idx, y * scores[idx, slots])
// which issues 3 launches per active expert and syncs on torch.where, with
// five stream-ordered launches and no host synchronisation:
//
//   1. route_kernel       one workgroup per two experts: counts of the ids
//                         equal to / below each expert, then a stable ballot
//                         compaction of the (token, slot) pairs routed to it
//                         in row-major order -- exactly torch.where's order.
//   2. quantize_rows      h (T, H) bf16 -> fp16-rounded -> MXFP4, once per
//                         token (the per-row quantization does not depend on
//                         which expert gathers the row).
//   3. grouped GEMM, gate/up   workgroup (feature tile, expert): for every
//                         128-token tile of the expert, A = gathered token
//                         rows, W = 64 gate rows + the same 64 up rows; the
//                         epilogue computes h = silu(g)*u in fp32, rounds it
//                         to fp16 (the x.to(half) of the `forward` binding)
//                         and quantizes it to MXFP4 in registers.
//   4. grouped GEMM, down      workgroup (output tile, expert): A = the
//                         expert's quantized h rows; the epilogue writes
//                         bf16(bf16(y) * score) per (token, slot) pair.
//   5. combine_kernel     out[t] = bf16(sum over the token's slots, fp32,
//                         slot order).  Ids outside [0, n_experts) contribute
//                         nothing, as an id missing from `experts` does in
//                         the reference.
//
// MFMA tiling is that of the lin_pq GEMM (128x128 tiles, K step 256, LDS
// double buffer, v_mfma_scale_f32_32x32x64_f8f6f4), with the operands
// swapped: the weight tile is the MFMA's A operand, so each lane ends with
// one token and 16 features of a 32-feature block.  The 32-block amax of h is
// then one exchange with lane l^32, and the nibbles pack into 8-byte stores.
#include <type_traits>

#include "lds_dma.h"
#include "mx_device.h"
#include "mx_host.h"
#include "quant_rows.h"

namespace mxh {
int quantize_rows_impl(const void* x, int src_dtype, int round_to_f16, int64_t ldx, int M, int K, int Kp,
                       uint8_t* q, uint8_t* s, hipStream_t st);
}

namespace {

constexpr int BM = 128, BN = 128, BK = 256;   // tokens, weight rows, K per step
constexpr int ROWB = BK / 2;
constexpr int LDSROW = ROWB + 16;
constexpr int SCB = BK / 32;
constexpr int TILE_BYTES = BM * LDSROW;
constexpr int BUF_BYTES = 2 * TILE_BYTES + 2 * BM * SCB;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopk = 32;

enum { MODE_GATEUP = 0, MODE_DOWN = 1 };

// ------------------------------------------------------------------ routing
// Workgroup b lists the pairs routed to experts 2b and 2b+1 (each id is
// read once per pass for two experts: half the traffic of one expert per
// workgroup, at twice the compare-and-ballot work per id, which is what
// bounds a workgroup here).  Each of the 8 waves owns a contiguous eighth of
// the row-major (token, slot) pairs: a first coalesced pass counts, per expert,
// its matches (ballot) and its valid ids below the first expert; the waves
// exchange the counts once through LDS; a second pass writes each expert's
// matches in order (ballot rank), so the result is a stable sort by expert
// id.  With `sscore`, the pair's routing weight is written beside it in
// sorted order (fp32 of the bf16 score), so the down epilogue needs no
// dependent load.
constexpr int kRouteEpw = 2;        // experts per workgroup
constexpr int kRouteWaves = 8;
__global__ __launch_bounds__(64 * kRouteWaves) void route_kernel(const int64_t* __restrict__ topi, int P, int n_exp,
                                                                 int* __restrict__ counts, int* __restrict__ offs,
                                                                 int* __restrict__ pairs,
                                                                 const uint16_t* __restrict__ scores,
                                                                 float* __restrict__ sscore) {
    __shared__ int s_eq[kRouteWaves][kRouteEpw], s_lt[kRouteWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int E0 = blockIdx.x * kRouteEpw;
    const int per_wave = ((P + 64 * kRouteWaves - 1) / (64 * kRouteWaves)) * 64;
    const int w0 = min(wave * per_wave, P);
    const int w1 = min(w0 + per_wave, P);
    constexpr int U = 16;  // chunks of 64 ids in flight per pass step (all of a wave's at P = 16384)
    int n_eq[kRouteEpw];
#pragma unroll
    for (int k = 0; k < kRouteEpw; ++k) n_eq[k] = 0;
    int n_lt = 0;
    for (int b = w0; b < w1; b += 64 * U) {
        int64_t id[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {   // clamped, unconditional loads: all U in flight at once
            const int p = b + 64 * u + lane;
            const int64_t v = topi[min(p, P - 1)];
            id[u] = p < w1 ? v : -1;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int k = 0; k < kRouteEpw; ++k)   // (ids >= n_exp match no expert)
                n_eq[k] += E0 + k < n_exp ? __popcll(__ballot(id[u] == (int64_t)(E0 + k))) : 0;
            n_lt += (id[u] >= 0 && id[u] < (int64_t)E0) ? 1 : 0;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) n_lt += __shfl_xor(n_lt, o);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < kRouteEpw; ++k) s_eq[wave][k] = n_eq[k];
        s_lt[wave] = n_lt;
    }
    __syncthreads();
    // expert E0+k starts after the valid ids below E0 and the matches of
    // E0 .. E0+k-1; this wave's matches of it after those of earlier waves
    int base = 0;
    for (int w = 0; w < kRouteWaves; ++w) base += s_lt[w];
    int pos[kRouteEpw];
#pragma unroll
    for (int k = 0; k < kRouteEpw; ++k) {
        int tot = 0, before = 0;
        for (int w = 0; w < kRouteWaves; ++w) {
            tot += s_eq[w][k];
            before += w < wave ? s_eq[w][k] : 0;
        }
        pos[k] = base + before;
        if (threadIdx.x == 0 && E0 + k < n_exp) {
            counts[E0 + k] = tot;
            offs[E0 + k] = base;
        }
        base += tot;
    }
    // second pass, in segments of 64*U ids: the wave's matches of the
    // segment, in order and grouped by expert, into its own LDS list, then
    // out with coalesced stores (one store per match would cost a memory
    // instruction per ballot)
    __shared__ int2 s_list[kRouteWaves][64 * U];
    int2* list = s_list[wave];
    for (int b = w0; b < w1; b += 64 * U) {
        int64_t id[U];
        uint16_t sc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int p = b + 64 * u + lane;
            const int64_t v = topi[min(p, P - 1)];
            id[u] = p < w1 ? v : -1;
            sc[u] = sscore ? scores[min(p, P - 1)] : (uint16_t)0;
        }
        int cnt[kRouteEpw], kb[kRouteEpw], rank[kRouteEpw];
        int kacc = 0;
#pragma unroll
        for (int k = 0; k < kRouteEpw; ++k) {
            cnt[k] = 0;
#pragma unroll
            for (int u = 0; u < U; ++u)
                cnt[k] += E0 + k < n_exp ? __popcll(__ballot(id[u] == (int64_t)(E0 + k))) : 0;
            kb[k] = kacc;
            kacc += cnt[k];
            rank[k] = 0;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int k = 0; k < kRouteEpw; ++k) {
                const bool m = E0 + k < n_exp && id[u] == (int64_t)(E0 + k);
                const unsigned long long bal = __ballot(m);
                if (m) list[kb[k] + rank[k] + __popcll(bal & ((1ull << lane) - 1ull))] = make_int2(b + 64 * u + lane, (int)sc[u]);
                rank[k] += __popcll(bal);
            }
        }
#pragma unroll
        for (int k = 0; k < kRouteEpw; ++k) {
            for (int q = lane; q < cnt[k]; q += 64) {
                const int2 v = list[kb[k] + q];
                pairs[pos[k] + q] = v.x;
                if (sscore) sscore[pos[k] + q] = mx::bf16_to_f32((uint16_t)v.y);
            }
            pos[k] += cnt[k];
        }
    }
}

// ------------------------------------------------------------------ routing, counting sort
// The same grouping (a stable sort of the row-major pairs by expert id) as a
// counting sort in two launches, whose work per id does not grow with the
// number of experts.  Chunks of kRtChunk ids; a wave takes 64 consecutive
// ids at a time and finds, for each lane, the lanes holding the same id with
// one ballot per id bit (the id's bits agree), so its rank among the equal
// ids of the 64 is a popcount.
//   route_count_kernel    chunk c: per-expert counts of its valid ids ->
//                         hist (nchunk, n_exp).
//   route_scatter_kernel  chunk c: expert e's pairs start at offs[e] (sum of
//                         the counts of ids below e) + the counts of e in
//                         chunks below c + in earlier waves of c + the
//                         earlier 64-id groups of the wave + the rank;
//                         writes pairs (and the sorted routing weights), and
//                         chunk 0 writes counts / offs.
constexpr int kRtWaves = 4;
constexpr int kRtGroups = 4;                          // 64-id groups per wave
constexpr int kRtChunk = 64 * kRtWaves * kRtGroups;   // 1024 ids per workgroup

__device__ __forceinline__ uint64_t same_id_lanes(int id, bool valid, int bits) {
    uint64_t m = __ballot(valid);
    for (int b = 0; b < bits; ++b) {
        const uint64_t s = __ballot((id >> b) & 1);
        m &= ((id >> b) & 1) ? s : ~s;
    }
    return m;
}

__device__ __forceinline__ int id_bits(int n_exp) { return 32 - __clz(max(n_exp - 1, 1)); }

// The token rows' quantization (x -> fp16 -> MXFP4) rides in the route
// count launch as the workgroups past its chunks: it does not depend on the
// routing, and the count's few latency-bound workgroups leave the CUs free.
struct XQuant {
    const void* x;      // (T, H) bf16
    int T, H;
    int lt, gx;         // quantize_rows_kernel's layout: 2^lt threads per row, gx row groups
    uint8_t* q;         // (T, H/2)
    uint8_t* s;         // (T, H/32)
};

__global__ __launch_bounds__(64 * kRtWaves) void route_count_kernel(const int64_t* __restrict__ topi, int P, int n_exp,
                                                                   int* __restrict__ hist, int* __restrict__ qctr,
                                                                   int nchunk, XQuant xq) {
    __shared__ int h[kMaxExperts];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if ((int)blockIdx.x >= nchunk) {
        const int local = (int)blockIdx.x - nchunk;
        const int bx = local % xq.gx, by = local / xq.gx;
        const int64_t row = (int64_t)bx * (256 >> xq.lt) + (tid >> xq.lt);
        const int u = by * (1 << xq.lt) + (tid & ((1 << xq.lt) - 1));
        mxq::quantize_unit<MXFP4_DT_BF16, 1>(xq.x, xq.H, xq.T, xq.H, xq.H, true, row, u, xq.q, xq.s);
        return;
    }
    if (qctr && blockIdx.x == 0 && tid < 16) qctr[tid] = 0;   // the grouped GEMMs' tile queues (8 each)
    for (int e = tid; e < n_exp; e += 64 * kRtWaves) h[e] = 0;
    const int bits = id_bits(n_exp);
    int id[kRtGroups];
#pragma unroll
    for (int k = 0; k < kRtGroups; ++k) {   // unconditional (clamped) loads: all in flight at once
        const int p = blockIdx.x * kRtChunk + (wave * kRtGroups + k) * 64 + lane;
        const int64_t v = topi[min(p, P - 1)];
        id[k] = (p < P && v >= 0 && v < n_exp) ? (int)v : -1;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kRtGroups; ++k) {
        const bool valid = id[k] >= 0;
        const uint64_t m = same_id_lanes(id[k], valid, bits);
        if (valid && (m & ((1ull << lane) - 1ull)) == 0) atomicAdd(&h[id[k]], __popcll(m));   // group leader
    }
    __syncthreads();
    for (int e = tid; e < n_exp; e += 64 * kRtWaves) hist[(int64_t)blockIdx.x * n_exp + e] = h[e];
}

__global__ __launch_bounds__(64 * kRtWaves) void route_scatter_kernel(const int64_t* __restrict__ topi, int P,
                                                                     int n_exp, const int* __restrict__ hist,
                                                                     int* __restrict__ counts, int* __restrict__ offs,
                                                                     int* __restrict__ pairs,
                                                                     const uint16_t* __restrict__ scores,
                                                                     float* __restrict__ sscore) {
    __shared__ int base[kMaxExperts];              // where expert e's pairs of this chunk start
    __shared__ int wh[kRtWaves][kMaxExperts];      // per-wave counts, then exclusive prefix over waves
    __shared__ int wsum[kRtWaves];
    __shared__ int carry;                          // running total of the scan over earlier slices
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nchunk = gridDim.x, c = blockIdx.x;
    if (tid == 0) carry = 0;
    const int bits = id_bits(n_exp);
    int id[kRtGroups];
    int64_t raw[kRtGroups];
    uint16_t sc[kRtGroups] = {};
    // all loads first (no use of a loaded value in between: one round trip)
#pragma unroll
    for (int k = 0; k < kRtGroups; ++k) raw[k] = topi[min(c * kRtChunk + (wave * kRtGroups + k) * 64 + lane, P - 1)];
    if (sscore) {
#pragma unroll
        for (int k = 0; k < kRtGroups; ++k) sc[k] = scores[min(c * kRtChunk + (wave * kRtGroups + k) * 64 + lane, P - 1)];
    }
#pragma unroll
    for (int k = 0; k < kRtGroups; ++k) {
        const int p = c * kRtChunk + (wave * kRtGroups + k) * 64 + lane;
        id[k] = (p < P && raw[k] >= 0 && raw[k] < n_exp) ? (int)raw[k] : -1;
    }
    // per expert: the total over all chunks and the count in chunks below c
    for (int e0 = 0; e0 < n_exp; e0 += 64 * kRtWaves) {
        const int e = e0 + tid;
        const int ec = min(e, n_exp - 1);
        int tot = 0, bef = 0;
        for (int cb = 0; cb < nchunk; cb += 16) {
            int v[16];   // 16 unconditional (clamped) loads in flight, then the sums
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = hist[(int64_t)min(cb + i, nchunk - 1) * n_exp + ec];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int x = (cb + i < nchunk && e < n_exp) ? v[i] : 0;
                tot += x;
                bef += cb + i < c ? x : 0;
            }
        }
        // exclusive scan of tot over e: waves, then the waves' sums
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o);
            if (lane >= o) incl += t;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();   // wsum, and carry from the previous slice
        int run = carry;
        for (int w = 0; w < wave; ++w) run += wsum[w];
        const int ex = run + incl - tot;
        if (e < n_exp) {
            base[e] = ex + bef;
            if (c == 0) {
                counts[e] = tot;
                offs[e] = ex;
            }
#pragma unroll
            for (int w = 0; w < kRtWaves; ++w) wh[w][e] = 0;
        }
        __syncthreads();   // every read of carry and wsum is done
        if (tid == 64 * kRtWaves - 1) carry = run + incl;   // read after the next slice's first barrier
    }
    __syncthreads();
    // this wave's counts per expert (group leaders; one writer per expert and group)
    uint64_t mk[kRtGroups];
#pragma unroll
    for (int k = 0; k < kRtGroups; ++k) {
        const bool valid = id[k] >= 0;
        mk[k] = same_id_lanes(id[k], valid, bits);
        if (valid && (mk[k] & ((1ull << lane) - 1ull)) == 0) wh[wave][id[k]] += __popcll(mk[k]);
    }
    __syncthreads();
    // exclusive prefix over the waves, per expert
    for (int e = tid; e < n_exp; e += 64 * kRtWaves) {
        int run = 0;
        for (int w = 0; w < kRtWaves; ++w) {
            const int v = wh[w][e];
            wh[w][e] = run;
            run += v;
        }
    }
    __syncthreads();
    // positions: the wave's earlier groups are counted in wh as it goes
#pragma unroll
    for (int k = 0; k < kRtGroups; ++k) {
        if (id[k] < 0) continue;
        const int at = base[id[k]] + wh[wave][id[k]] + __popcll(mk[k] & ((1ull << lane) - 1ull));
        const int p = c * kRtChunk + (wave * kRtGroups + k) * 64 + lane;
        pairs[at] = p;
        if (sscore) sscore[at] = mx::bf16_to_f32(sc[k]);
        // after every lane has its position, the group leader moves the
        // wave's offset of this expert past the group
        if ((mk[k] & ((1ull << lane) - 1ull)) == 0) wh[wave][id[k]] += __popcll(mk[k]);
    }
}

// ------------------------------------------------------------------ weights
struct StackedW {                // expert e of projection j at base[j] + e * stride
    const uint8_t* wp[3];
    const uint8_t* ws[3];
    int64_t wp_stride[3], ws_stride[3];
    __device__ const uint8_t* p(int e, int j) const { return wp[j] + (int64_t)e * wp_stride[j]; }
    __device__ const uint8_t* s(int e, int j) const { return ws[j] + (int64_t)e * ws_stride[j]; }
};
struct TableW {                  // device table (n_experts, 6) int64: gate wp/ws, up wp/ws, down wp/ws
    const int64_t* tab;
    __device__ const uint8_t* p(int e, int j) const { return reinterpret_cast<const uint8_t*>(tab[e * 6 + 2 * j]); }
    __device__ const uint8_t* s(int e, int j) const { return reinterpret_cast<const uint8_t*>(tab[e * 6 + 2 * j + 1]); }
};

struct GArgs {
    const uint8_t* aq;       // GATEUP: token rows (T, H/2); DOWN: sorted h rows (P, Mi/2)
    const uint8_t* as;       // matching scale rows
    const int* counts;
    const int* offs;
    const int* pairs;
    int topk;
    int Kp;                  // K of this GEMM: H (gate/up) or Mi (down)
    int Nw;                  // weight rows per projection: Mi (gate/up) or H (down)
    uint8_t* hq;             // GATEUP out: (P, Mi/2) MXFP4 h in sorted order
    uint8_t* hs;             //             (P, Mi/32)
    uint16_t* yd;            // DOWN out: (P, H) bf16 at the pair's own index
    const float* sscore;     // DOWN: (P) routing weights in sorted pair order
    int a_rows;              // rows of aq / as (T for gate/up, P for down)
};

struct StageRegs {
    uint4 a[4];
    uint4 w[4];
    uint2 sc;
};

// One K step: 4 x 16 B of A rows and of W rows per thread, 8 scale bytes of
// one row (threads 0..127: A row, 128..255: W row).  Row base pointers are
// resolved once per token tile (gathered tokens, gate/up interleave).
__device__ __forceinline__ void load_stage(StageRegs& r, const uint8_t* const arow[4], const uint8_t* const wrow[4],
                                           const uint8_t* srow, int Kp, int k0) {
    const int tid = threadIdx.x;
    const int nch = Kp >> 5;
    const int kb0 = k0 >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ch = tid & 7;
        const bool kok = kb0 + ch < nch;
        const int off = (k0 >> 1) + ch * 16;
        r.a[i] = kok ? *reinterpret_cast<const uint4*>(arow[i] + off) : make_uint4(0, 0, 0, 0);
        r.w[i] = kok ? *reinterpret_cast<const uint4*>(wrow[i] + off) : make_uint4(0, 0, 0, 0);
    }
    const uint8_t* sp = srow + kb0;
    if (kb0 + SCB <= nch && (((uintptr_t)sp) & 7) == 0) {
        r.sc = *reinterpret_cast<const uint2*>(sp);
    } else {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < SCB; ++j) {
            const uint32_t b = (kb0 + j < nch) ? (uint32_t)sp[j] : 127u;
            if (j < 4) lo |= b << (8 * j);
            else hi |= b << (8 * (j - 4));
        }
        r.sc = make_uint2(lo, hi);
    }
}

__device__ __forceinline__ void store_stage(const StageRegs& r, uint8_t* buf) {
    const int tid = threadIdx.x;
    uint8_t* la = buf;
    uint8_t* lw = buf + TILE_BYTES;
    uint8_t* lsa = buf + 2 * TILE_BYTES;
    uint8_t* lsw = lsa + BM * SCB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = (tid >> 3) + 32 * i;
        const int ch = tid & 7;
        *reinterpret_cast<uint4*>(la + row * LDSROW + ch * 16) = r.a[i];
        *reinterpret_cast<uint4*>(lw + row * LDSROW + ch * 16) = r.w[i];
    }
    const int row = tid & 127;
    *reinterpret_cast<uint2*>((tid >= 128 ? lsw : lsa) + row * SCB) = r.sc;
}

__device__ __forceinline__ uint32_t scale_word(const uint8_t* srow, int h) {
    const uint2 v = *reinterpret_cast<const uint2*>(srow);
    return __builtin_amdgcn_perm(v.y, v.x, h ? 0x07050301u : 0x06040200u);
}

template <int OP>
__device__ __forceinline__ mx::v16f mfma32(uint4 a, uint4 b, mx::v16f c, uint32_t sa, uint32_t sb) {
    mx::v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    mx::v8i bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 4, 4, OP, (int)sa, OP, (int)sb);
}

// Weight row of tile row rho (0..127).  Gate/up: rows [32b, 32b+32) hold
// projection b&1 (0 gate, 1 up) of features f0 + 32*(b>>1) + 0..31, so a
// wave's two 32-row blocks are the gate and up rows of the same features.
template <int MODE>
__device__ __forceinline__ int weight_row(int rho, int n0, int& proj) {
    if (MODE == MODE_GATEUP) {
        const int b = rho >> 5;
        proj = b & 1;
        return n0 + 32 * (b >> 1) + (rho & 31);
    }
    proj = 2;
    return n0 + rho;
}

// Down epilogue inputs of the lane's two token rows rbase + 32i + lr: the
// pair index and its routing weight (loaded ahead of the K loop by the
// kernels that can, so the epilogue waits on no load).
__device__ __forceinline__ void down_rows(const GArgs& g, int off, int mt, int mrows, int rbase, int lr, int (&pp)[2],
                                          float (&ss)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rloc = rbase + 32 * i + lr;
        pp[i] = rloc < mrows ? g.pairs[off + mt + rloc] : 0;
        ss[i] = rloc < mrows ? g.sscore[off + mt + rloc] : 0.0f;
    }
}

// Epilogue of a 128 x 128 tile (acc[i][j] of the 2 x 2 wave layout):
// gate/up -> h = silu(g)*u, fp16, MXFP4 rows in sorted pair order; down ->
// bf16(bf16(y) * score) at the pair's own index (pp / ss from down_rows).
// NI: how many of the two token blocks to process (1: only acc[0]).
template <int MODE, int NI = 2>
__device__ __forceinline__ void tile_epilogue(mx::v16f (&acc)[2][2], const GArgs& g, int n0, int off, int mt,
                                              int mrows, int rbase, int wn, int lr, int h, const int (&pp)[2],
                                              const float (&ss)[2], int istride = 32) {
    // acc[i][j] element q of lane l: token rbase + istride*i + l%32, weight
    // row wn*64 + 32j + 8(q/4) + 4h + q%4 of the tile
    if (MODE == MODE_GATEUP) {
        const int fb = n0 + 32 * wn;           // first feature of this wave's 32-block
        const int Mi = g.Nw;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int rloc = rbase + istride * i + lr;
            float v[16];
            float amax = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                v[q] = mx::round_to_f16(mx::silu_mul_fast(acc[i][0][q], acc[i][1][q]));
                amax = fmaxf(amax, fabsf(v[q]));
            }
            amax = fmaxf(amax, __shfl_xor(amax, 32));
            const uint32_t code = mx::e8m0_code(amax);
            const float inv = mx::e8m0_inv_scale(code);
            uint32_t piece[4];   // v is exact in fp16: the hardware codes (mx::e2m1_hw_arg)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                piece[q4] = mx::e2m1_hw_pair<0>(0u, v[4 * q4] * inv, v[4 * q4 + 1] * inv);
                piece[q4] = mx::e2m1_hw_pair<1>(piece[q4], v[4 * q4 + 2] * inv, v[4 * q4 + 3] * inv);
            }
            // lane h holds features 8*q4 + 4h + 0..3 -> bytes 4*q4 + 2h, +1
            const uint32_t send = h ? (piece[0] | (piece[1] << 16)) : (piece[2] | (piece[3] << 16));
            const uint32_t recv = __shfl_xor(send, 32);
            uint2 d;
            if (h == 0) {
                d.x = piece[0] | ((recv & 0xFFFFu) << 16);
                d.y = piece[1] | ((recv >> 16) << 16);
            } else {
                d.x = (recv & 0xFFFFu) | (piece[2] << 16);
                d.y = (recv >> 16) | (piece[3] << 16);
            }
            if (rloc < mrows && fb < Mi) {
                const int64_t srow_i = off + mt + rloc;
                *reinterpret_cast<uint2*>(g.hq + srow_i * (Mi >> 1) + (fb >> 1) + 8 * h) = d;
                if (h == 0) g.hs[srow_i * (Mi >> 5) + (fb >> 5)] = (uint8_t)code;
            }
        }
    } else {
        const int H = g.Nw;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int rloc = rbase + istride * i + lr;
            if (rloc < mrows) {
                const int p = pp[i];
                const float sc = ss[i];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int cb = n0 + wn * 64 + 32 * j;   // 32-column block
                    if (cb < H) {
#pragma unroll
                        for (int q4 = 0; q4 < 4; ++q4) {
                            uint32_t b[2];
#pragma unroll
                            for (int r = 0; r < 2; ++r) {
                                // bf16(bf16(y) * score), two at a time
                                const uint32_t y2 = mx::f32x2_to_bf16x2(acc[i][j][4 * q4 + 2 * r], acc[i][j][4 * q4 + 2 * r + 1]);
                                b[r] = mx::f32x2_to_bf16x2(__uint_as_float(y2 << 16) * sc,
                                                           __uint_as_float(y2 & 0xFFFF0000u) * sc);
                            }
                            *reinterpret_cast<uint2*>(g.yd + (int64_t)p * H + cb + 8 * q4 + 4 * h) = make_uint2(b[0], b[1]);
                        }
                    }
                }
            }
        }
    }
}

template <int MODE, class W>
__global__ __launch_bounds__(256, 2) void grouped_gemm_kernel(GArgs g, W w) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int e = blockIdx.y;
    const int cnt = g.counts[e];
    if (cnt == 0) return;
    const int off = g.offs[e];
    // gate/up: 64 features per workgroup; down: 128 output columns
    const int n0 = blockIdx.x * (MODE == MODE_GATEUP ? BN / 2 : BN);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31;
    const int h = lane >> 5;
    const int cbytes = g.Kp >> 1;
    const int nch = g.Kp >> 5;
    const int nsteps = (g.Kp + BK - 1) / BK;

    // weight rows of this thread (fixed for the whole workgroup)
    const uint8_t* wrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int proj;
        const int rr = min(weight_row<MODE>((tid >> 3) + 32 * i, n0, proj), g.Nw - 1);
        wrow[i] = w.p(e, proj) + (int64_t)rr * cbytes;
    }
    const uint8_t* wsrow;
    {
        int proj;
        const int rr = min(weight_row<MODE>(tid & 127, n0, proj), g.Nw - 1);
        wsrow = w.s(e, proj) + (int64_t)rr * nch;
    }

    for (int mt = 0; mt < cnt; mt += BM) {
        const int mrows = min(BM, cnt - mt);
        // token (A) rows of this thread, clamped to the tile's last valid row
        const uint8_t* arow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = min((tid >> 3) + 32 * i, mrows - 1);
            const int src = MODE == MODE_GATEUP ? g.pairs[off + mt + r] / g.topk : off + mt + r;
            arow[i] = g.aq + (int64_t)src * cbytes;
        }
        const uint8_t* srow = wsrow;
        if (tid < 128) {
            const int r = min(tid, mrows - 1);
            const int src = MODE == MODE_GATEUP ? g.pairs[off + mt + r] / g.topk : off + mt + r;
            srow = g.as + (int64_t)src * nch;
        }

        mx::v16f acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

        StageRegs st;
        load_stage(st, arow, wrow, srow, g.Kp, 0);
        store_stage(st, smem);
        __syncthreads();
        for (int it = 0; it < nsteps; ++it) {
            uint8_t* cur = smem + (it & 1) * BUF_BYTES;
            const bool more = it + 1 < nsteps;
            if (more) load_stage(st, arow, wrow, srow, g.Kp, (it + 1) * BK);
            const uint8_t* la = cur;
            const uint8_t* lw = cur + TILE_BYTES;
            const uint8_t* lsa = cur + 2 * TILE_BYTES;
            const uint8_t* lsw = lsa + BM * SCB;
            uint32_t sa[2], sb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                sa[i] = scale_word(lsa + (wm * 64 + i * 32 + lr) * SCB, h);
                sb[i] = scale_word(lsw + (wn * 64 + i * 32 + lr) * SCB, h);
            }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                uint4 af[2], bf[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    af[i] = *reinterpret_cast<const uint4*>(la + (wm * 64 + i * 32 + lr) * LDSROW + ks * 32 + h * 16);
                    bf[i] = *reinterpret_cast<const uint4*>(lw + (wn * 64 + i * 32 + lr) * LDSROW + ks * 32 + h * 16);
                }
                // D[weight row][token]: the weight tile is the MFMA A operand
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (ks == 0) acc[i][j] = mfma32<0>(bf[j], af[i], acc[i][j], sb[j], sa[i]);
                        if (ks == 1) acc[i][j] = mfma32<1>(bf[j], af[i], acc[i][j], sb[j], sa[i]);
                        if (ks == 2) acc[i][j] = mfma32<2>(bf[j], af[i], acc[i][j], sb[j], sa[i]);
                        if (ks == 3) acc[i][j] = mfma32<3>(bf[j], af[i], acc[i][j], sb[j], sa[i]);
                    }
            }
            if (more) store_stage(st, smem + ((it + 1) & 1) * BUF_BYTES);
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) mx::pin(acc[i][j]);

        int pp[2] = {0, 0};
        float ss[2] = {0.0f, 0.0f};
        if (MODE == MODE_DOWN) down_rows(g, off, mt, mrows, wm * 64, lr, pp, ss);
        tile_epilogue<MODE>(acc, g, n0, off, mt, mrows, wm * 64, wn, lr, h, pp, ss);
        __syncthreads();   // LDS buffers are refilled by the next token tile
    }
}

// ------------------------------------------------------------------ LDS-copy ring variant
// Tiles of 256 tokens x 128 weight rows (a wave: 128 tokens x 64 rows), so an
// expert's ~128-250 routed tokens take one pass over its weights: with
// 128-token tiles half of the experts streamed their weights twice, the
// second time for a handful of tokens.  The operands are copied global ->
// LDS by buffer_load ... lds (no registers) into a ring of D_NST stages of
// 128-wide K slices, two slices of copies in flight while a third is
// multiplied.  LDS rows are 64 bytes with an XOR swizzle of their four
// 16-byte chunks, so the 16 lanes of an operand read hit distinct bank
// groups.  The epilogues are the 128 x 128 kernel's.  Requires Kp % 128 == 0.
constexpr int DM = 256;                     // tokens per tile
constexpr int DK = 128;                     // K per stage
constexpr int DROWB = DK / 2;               // bytes per row per stage
constexpr int D_A = DM * DROWB;             // 16 KB of token rows
constexpr int D_W = BN * DROWB;             // 8 KB of weight rows
constexpr int D_SA = DM * 4;                // 4 scale bytes per row
constexpr int D_SW = BN * 4;
constexpr int D_STAGE = D_A + D_W + D_SA + D_SW;
constexpr int D_NST = 3;
constexpr int D_COPIES = 8;                 // per wave per stage: 4 token-row, 2 weight-row, 2 scale copies

__device__ __forceinline__ int dswz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

__device__ __forceinline__ uint32_t scale4(const uint8_t* p, int h) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
    return __builtin_amdgcn_perm(v, v, h ? 0x0C0C0301u : 0x0C0C0200u);   // byte ks = block 2ks + h
}

template <int MODE, class W>
__global__ __launch_bounds__(256, 2) void grouped_gemm_dma_kernel(GArgs g, W w) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int e = blockIdx.y;
    const int cnt = g.counts[e];
    if (cnt == 0) return;
    const int off = g.offs[e];
    const int n0 = blockIdx.x * (MODE == MODE_GATEUP ? BN / 2 : BN);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31;
    const int h = lane >> 5;
    const uint32_t cbytes = (uint32_t)g.Kp >> 1, nch = (uint32_t)g.Kp >> 5;
    const int nsteps = g.Kp / DK;
    const uint32_t ring = __builtin_amdgcn_readfirstlane(mx::lds_addr(smem));
    const int slot = lane & 3;

    // weight-row copies: 1 KB blocks 2*wave, 2*wave+1 of the W tile (16 rows
    // each, all of one projection: projections change every 32 rows)
    mx::v4u wrs[2];
    uint32_t wvo[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int rho = 16 * (2 * wave + j) + (lane >> 2);
        int proj;
        const int rr = min(weight_row<MODE>(rho, n0, proj), g.Nw - 1);
        wrs[j] = mx::buf_rsrc(w.p(e, proj), (int64_t)g.Nw * cbytes);
        wvo[j] = (uint32_t)rr * cbytes + ((slot ^ dswz(rho)) << 4);
    }
    // scale copies: wave w copies the token rows' scales of rows 64w..64w+63
    // and (lanes 0..31) the weight rows' of rows 32w..32w+31, one projection
    uint32_t svo_w;
    int wproj;
    {
        const int rr = min(weight_row<MODE>(32 * wave + (lane & 31), n0, wproj), g.Nw - 1);
        svo_w = (uint32_t)rr * nch;
    }
    const mx::v4u srs_w = mx::buf_rsrc(w.s(e, wproj), (int64_t)g.Nw * nch);
    const mx::v4u ars = mx::buf_rsrc(g.aq, (int64_t)g.a_rows * cbytes);
    const mx::v4u asrs = mx::buf_rsrc(g.as, (int64_t)g.a_rows * nch);

    for (int mt = 0; mt < cnt; mt += DM) {
        const int mrows = min(DM, cnt - mt);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the previous tile's stores
        uint32_t avo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ra = 16 * (4 * wave + j) + (lane >> 2);
            const int r = min(ra, mrows - 1);
            const int src = MODE == MODE_GATEUP ? g.pairs[off + mt + r] / g.topk : off + mt + r;
            avo[j] = (uint32_t)src * cbytes + ((slot ^ dswz(ra)) << 4);
        }
        uint32_t svo_a;
        {
            const int r = min(64 * wave + lane, mrows - 1);
            const int src = MODE == MODE_GATEUP ? g.pairs[off + mt + r] / g.topk : off + mt + r;
            svo_a = (uint32_t)src * nch;
        }

        auto issue = [&](int stg, int k) {
            const uint32_t buf = ring + stg * D_STAGE;
            const uint32_t kofs = (uint32_t)k * DROWB;
#pragma unroll
            for (int j = 0; j < 4; ++j) mx::dma16(avo[j], ars, kofs, buf + (4 * wave + j) * 1024);
#pragma unroll
            for (int j = 0; j < 2; ++j) mx::dma16(wvo[j], wrs[j], kofs, buf + D_A + (2 * wave + j) * 1024);
            const uint32_t ksc = (uint32_t)k * 4;
            mx::dma4(svo_a, asrs, ksc, buf + D_A + D_W + 256 * wave);
            if (lane < 32) mx::dma4(svo_w, srs_w, ksc, buf + D_A + D_W + D_SA + 128 * wave);
        };

        mx::v16f acc[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

#pragma unroll
        for (int st = 0; st < D_NST - 1; ++st) issue(st, min(st, nsteps - 1));
        const int key = dswz(lr);
        for (int it = 0; it < nsteps; ++it) {
            // this wave's copies of step it have landed (later steps' may still
            // be in flight) and its reads of step it-1 are done; after the
            // barrier every wave's.  Past the last step the copies re-read the
            // last slice, so every step has the same count outstanding.
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((D_NST - 2) * D_COPIES) : "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            issue((it + D_NST - 1) % D_NST, min(it + D_NST - 1, nsteps - 1));
            const uint8_t* cur = smem + (it % D_NST) * D_STAGE;
            const uint8_t* la = cur;
            const uint8_t* lw = cur + D_A;
            const uint8_t* lsa = cur + D_A + D_W;
            const uint8_t* lsw = lsa + D_SA;
            uint32_t sa[4], sb[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) sa[i] = scale4(lsa + (wm * 128 + i * 32 + lr) * 4, h);
#pragma unroll
            for (int j = 0; j < 2; ++j) sb[j] = scale4(lsw + (wn * 64 + j * 32 + lr) * 4, h);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int koff = ((2 * ks + h) ^ key) << 4;
                uint4 af[4], bf[2];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    af[i] = *reinterpret_cast<const uint4*>(la + (wm * 128 + i * 32 + lr) * DROWB + koff);
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    bf[j] = *reinterpret_cast<const uint4*>(lw + (wn * 64 + j * 32 + lr) * DROWB + koff);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (ks == 0) acc[i][j] = mfma32<0>(bf[j], af[i], acc[i][j], sb[j], sa[i]);
                        if (ks == 1) acc[i][j] = mfma32<1>(bf[j], af[i], acc[i][j], sb[j], sa[i]);
                    }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the copies issued past the last step
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) mx::pin(acc[i][j]);
        // the wave's 128 token rows as two 64-row halves of the 128 x 128 epilogue
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            mx::v16f sub[2][2] = {{acc[2 * half][0], acc[2 * half][1]}, {acc[2 * half + 1][0], acc[2 * half + 1][1]}};
            int pp[2] = {0, 0};
            float ss[2] = {0.0f, 0.0f};
            if (MODE == MODE_DOWN) down_rows(g, off, mt, mrows, wm * 128 + 64 * half, lr, pp, ss);
            tile_epilogue<MODE>(sub, g, n0, off, mt, mrows, wm * 128 + 64 * half, wn, lr, h, pp, ss);
        }
        __syncthreads();   // the ring is refilled by the next token tile
    }
}

// ------------------------------------------------------------------ 192 x 256 tiles, 8 waves
// Tiles of up to 192 tokens x 256 weight rows (gate/up: the gate and up rows
// of 128 features; down: 256 output columns), 8 waves in 2 (tokens) x 4
// (weight rows), a wave owning up to 3 x 2 MFMA accumulators.  K step 256,
// so every copied row piece is a whole 128-byte line (global -> LDS by
// buffer_load ... lds, XOR swizzle of the 16-byte chunks).  The weight rows,
// which stream from HBM, sit in a 3-stage ring and the token rows, which
// mostly hit L2, in a 2-stage ring: during step k the copies of the token
// rows of step k+1 and of the weight rows of step k+2 are in flight, in that
// order, so the wait at the top of step k+1 leaves the last five copies (the
// weights of step k+2) outstanding.  One workgroup per CU (156 KB of LDS).
//  * The token tile is sized to the expert's count in 64-row steps (only
//    ceil(rows / 64) * 64 token rows are copied), and a wave issues the MFMAs
//    of only those of its 32-token blocks that hold routed tokens, so an
//    expert with ~130 tokens costs what ~130 tokens need.  Token block i of
//    wave (wm, wn) is tile block 2i + wm: the two waves of a SIMD share the
//    routed rows, so each one's MFMAs run while the other waits on its
//    operand reads, which are issued one MFMA substep ahead.
//  * All tiles of one expert run on workgroups of one residue mod 8, i.e.
//    on one XCD (workgroups are dealt to the 8 XCDs round-robin), so the
//    expert's gathered token rows are fetched into one L2.
// Requires Kp % 256 == 0.
constexpr int X_BM = 192, X_BN = 256;
constexpr int X_ROWB = 128;                           // bytes per row per K step
constexpr int X_A = X_BM * X_ROWB;                    // 24 KB of token rows
constexpr int X_W = X_BN * X_ROWB;                    // 32 KB of weight rows
constexpr int X_AST = X_A + X_BM * 8;                 // token stage: rows + 8 scale bytes per row
constexpr int X_WST = X_W + X_BN * 8;                 // weight stage
constexpr int X_ARING = 3 * X_WST;                    // the token ring follows the 3-stage weight ring
constexpr int X_THREADS = 512;
constexpr int X_PP = X_ARING + 2 * X_AST;             // the down tile's pair indices and weights
constexpr int X_LDS = X_PP + 8 * X_BM;
static_assert(X_LDS <= 160 * 1024, "x8 LDS layout");

// Per-tile copy plan of one wave: na token-row blocks (8 rows of 128 bytes
// each), 4 weight-row blocks, one weight-scale copy (32 rows x 8 bytes) and,
// for waves < 2 na, one token-scale copy.
struct XCopies {
    mx::v4u ars, wrs, sars, swrs;
    uint32_t avo[3], wvo[4], savo, swvo;
    int na;
};

// Source rows of a wave's copies of one token tile: the rows of its three
// token-row blocks (64j + 8*wave + lane/8) and of its token-scale copy
// (32*wave + lane/2), clamped to the tile.  Gate/up: the sorted pair index
// (the token is it / topk, taken by x8_plan_rows); down: the sorted h row.
template <int MODE>
__device__ __forceinline__ void x8_rows(int (&rw)[4], const GArgs& g, int off, int mt, int mrows, int wave, int lane) {
    auto src = [&](int r) {
        const int rc = min(r, mrows - 1);
        return MODE == MODE_GATEUP ? g.pairs[off + mt + rc] : off + mt + rc;
    };
#pragma unroll
    for (int j = 0; j < 3; ++j) rw[j] = src(64 * j + 8 * wave + (lane >> 3));
    rw[3] = src(32 * wave + (lane >> 1));
}

template <int MODE, class W>
__device__ __forceinline__ void x8_plan_rows(XCopies& c, const GArgs& g, const W& w, int e, int n0, int mrows,
                                             const int (&rw)[4], int wave, int lane) {
    const uint32_t cbytes = (uint32_t)g.Kp >> 1, nch = (uint32_t)g.Kp >> 5;
    const int slot = lane & 7;
    c.na = (mrows + 63) >> 6;
    auto row_of = [&](int v) { return MODE == MODE_GATEUP ? v / g.topk : v; };
    c.ars = mx::buf_rsrc(g.aq, (int64_t)g.a_rows * cbytes);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int r = 64 * j + 8 * wave + (lane >> 3);   // block 8j + wave
        c.avo[j] = (uint32_t)row_of(rw[j]) * cbytes + ((slot ^ mx::swz_key128(r)) << 4);
    }
    // weight blocks 4*wave + j: rows 32*wave .. +31, one projection
    int proj;
    weight_row<MODE>(32 * wave, n0, proj);
    c.wrs = mx::buf_rsrc(w.p(e, proj), (int64_t)g.Nw * cbytes);
    c.swrs = mx::buf_rsrc(w.s(e, proj), (int64_t)g.Nw * nch);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int rho = 32 * wave + 8 * j + (lane >> 3);
        int pj;
        const int rr = min(weight_row<MODE>(rho, n0, pj), g.Nw - 1);
        c.wvo[j] = (uint32_t)rr * cbytes + ((slot ^ mx::swz_key128(rho)) << 4);
    }
    {   // scale copies: lane -> row 32 * wave + lane / 2, 4 of its 8 bytes
        const int row = 32 * wave + (lane >> 1);
        int pj;
        const int rr = min(weight_row<MODE>(row, n0, pj), g.Nw - 1);
        c.swvo = (uint32_t)rr * nch + 4 * (lane & 1);
        c.sars = mx::buf_rsrc(g.as, (int64_t)g.a_rows * nch);
        c.savo = (uint32_t)row_of(rw[3]) * nch + 4 * (lane & 1);
    }
}

// The token-row copies of K step s into the token stage at `abuf`, part
// `part` (parts 0-1), and the weight-row copies of step s into the weight
// stage at `wbuf`, part `part` (parts 2-3): within a step all token copies
// come first and the last five are the weight copies.
__device__ __forceinline__ void x8_issue_a(const XCopies& c, uint32_t abuf, int s, int part, int wave) {
    const uint32_t kofs = (uint32_t)s * X_ROWB;
    if (part == 0) {
        if (c.na > 0) mx::dma16(c.avo[0], c.ars, kofs, abuf + wave * 1024);
        if (c.na > 1) mx::dma16(c.avo[1], c.ars, kofs, abuf + (8 + wave) * 1024);
        if (wave < 2 * c.na) mx::dma4(c.savo, c.sars, (uint32_t)s * 8, abuf + X_A + 256 * wave);
    } else if (c.na > 2) {
        mx::dma16(c.avo[2], c.ars, kofs, abuf + (16 + wave) * 1024);
    }
}
__device__ __forceinline__ void x8_issue_w(const XCopies& c, uint32_t wbuf, int s, int part, int wave) {
    const uint32_t kofs = (uint32_t)s * X_ROWB;
    const int j0 = 2 * (part - 2);
    mx::dma16(c.wvo[j0], c.wrs, kofs, wbuf + (4 * wave + j0) * 1024);
    mx::dma16(c.wvo[j0 + 1], c.wrs, kofs, wbuf + (4 * wave + j0 + 1) * 1024);
    if (part == 2) mx::dma4(c.swvo, c.swrs, (uint32_t)s * 8, wbuf + X_W + 256 * wave);
}

// ------------------------------------------------------------------ persistent 192 x 256 tiles
// grouped_gemm_xp_kernel<MODE>: the tiles above, with one workgroup per CU
// that takes tiles from its group's queue until the queue is empty.  A
// tile's plan and first copies (weights of steps 0 and 1, tokens of step 0)
// are issued during the previous tile's epilogue, so they land while that
// epilogue runs instead of after one workgroup has exited and the next has
// started (a workgroup per tile, one per CU: 140 us per config-3b call
// against 133 us).
//  * Groups: workgroup b is in group b % 8, i.e. on XCD b % 8 (workgroups
//    are dealt to the XCDs round-robin), and group x computes the experts
//    e = x, x+8, ..., so an expert's token rows are fetched into one L2.
//  * Units: a group's tiles are (expert j, token tile, weight-row tile),
//    expert-major, then token tile, then weight-row tile, so the weight-row
//    tiles of an expert run at about the same time and share its token rows.
//    At the start every workgroup counts its group's units from the expert
//    counts (a prefix over the group's experts, in LDS); a unit index names
//    its tile by a ballot over the prefix.  Workgroup k of a group (of P)
//    takes units k and k + P first; the group's queue (an atomic counter the
//    route kernel zeroes) hands out the rest from 2P on, one per tile and a
//    tile ahead, so the next tile is known when a tile starts and its source
//    rows load during the K loop.
//  * The weight ring is used from stage 1 on (K step s in stage (s+1) % 3):
//    the down epilogue transposes its blocks in stage 0, which the next tile
//    first refills during its step 0, after the barrier every wave reaches
//    only past its epilogue.  The next tile's copies go to stages 1 and 2
//    and token stage 0, read by no wave once all are past the last K step.
//  * Waits: the copies are invisible to the compiler (inline asm), so a load
//    whose value is used while copies are in flight would make it wait for
//    all of them.  The loads of a tile (the next tile's source rows, the
//    queue atomic, the down tile's pair indices and weights) are issued at
//    its start and used only after its K loop, where no copy is in flight.
constexpr int XP_TROW = 136;                                // down transpose: 128 B + 8 per row
static_assert(8 * 32 * XP_TROW <= X_WST, "the down transposes fit weight stage 0");
constexpr int XP_MAXJ = kMaxExperts / 8;                    // experts per group
constexpr int XP_UCUM = X_LDS;                              // int[XP_MAXJ + 1]: units of the experts below j
constexpr int XP_ECNT = XP_UCUM + 4 * (XP_MAXJ + 1);        // int[XP_MAXJ]: expert counts
constexpr int XP_EOFF = XP_ECNT + 4 * XP_MAXJ;              // int[XP_MAXJ]: expert offsets
constexpr int XP_SLOT = XP_EOFF + 4 * XP_MAXJ;              // int: the unit the queue handed out
constexpr int XP_LDS = XP_SLOT + 16;
static_assert(XP_LDS <= 160 * 1024 && XP_MAXJ <= 128, "xp LDS layout (two experts per lane in the prefix)");

struct XpTile {
    int e, n0, off, mt, mrows;
};

// The tile of unit u (uniform): the expert j of the group with
// ucum[j] <= u < ucum[j+1], found by a ballot over the group's experts.
template <int MODE>
__device__ __forceinline__ XpTile xp_tile_of(const uint8_t* smem, int grp, int nj, int ntiles, int u, int lane) {
    const int* ucum = reinterpret_cast<const int*>(smem + XP_UCUM);
    int j = 0;
    for (int b = 0; b < nj; b += 64) {
        const int jj = b + lane;
        const bool hit = jj < nj && ucum[jj] <= u && u < ucum[jj + 1];
        const uint64_t m = __ballot(hit);
        if (m) {
            j = b + __ffsll((unsigned long long)m) - 1;
            break;
        }
    }
    j = __builtin_amdgcn_readfirstlane(j);
    const int local = u - ucum[j];
    const int mti = local / ntiles;
    const int nt = local - mti * ntiles;
    XpTile t;
    t.e = grp + 8 * j;
    t.off = __builtin_amdgcn_readfirstlane(reinterpret_cast<const int*>(smem + XP_EOFF)[j]);
    const int cnt = __builtin_amdgcn_readfirstlane(reinterpret_cast<const int*>(smem + XP_ECNT)[j]);
    t.mt = __builtin_amdgcn_readfirstlane(mti * X_BM);
    t.mrows = min(X_BM, cnt - t.mt);
    t.n0 = __builtin_amdgcn_readfirstlane(nt * (MODE == MODE_GATEUP ? X_BN / 2 : X_BN));
    return t;
}

// A tile's first copies in three parts, in the order the K loop's waits
// count on: 0, the weights of step 0 (stage 1); 1, the tokens of step 0;
// 2, the weights of step 1 (stage 2).  Before part 0 the plan's offsets and
// descriptors pass through an empty asm, so that they (and the compiler's
// waits for the plan's loads) are complete before the first copy is
// issued: a wait placed after a copy would also wait for the copy, which
// the compiler does not count.
__device__ __forceinline__ void xp_prologue_part(XCopies& c, uint32_t ring, int nsteps, int wave, int part) {
    if (part == 0) {
        asm volatile("" : "+v"(c.avo[0]), "+v"(c.avo[1]), "+v"(c.avo[2]), "+v"(c.savo), "+v"(c.wvo[0]),
                     "+v"(c.wvo[1]), "+v"(c.wvo[2]), "+v"(c.wvo[3]), "+v"(c.swvo), "+s"(c.ars), "+s"(c.wrs),
                     "+s"(c.sars), "+s"(c.swrs) :: "memory");
        x8_issue_w(c, ring + X_WST, 0, 2, wave);
        x8_issue_w(c, ring + X_WST, 0, 3, wave);
    } else if (part == 1) {
        x8_issue_a(c, ring + X_ARING, 0, 0, wave);
        x8_issue_a(c, ring + X_ARING, 0, 1, wave);
    } else if (nsteps > 1) {
        x8_issue_w(c, ring + 2 * X_WST, 1, 2, wave);
        x8_issue_w(c, ring + 2 * X_WST, 1, 3, wave);
    }
}

__device__ __forceinline__ void xp_prologue(XCopies& c, uint32_t ring, int nsteps, int wave) {
    for (int part = 0; part < 3; ++part) xp_prologue_part(c, ring, nsteps, wave, part);
}

template <int MODE, int NB, class Issue>
__device__ __forceinline__ void xp_epilogue(mx::v16f (&acc)[3][2], const GArgs& g, uint8_t* smem, const XpTile& t,
                                            int wave, int lane, Issue&& issue);

// K loop of one wave on tile t (its prologue already issued), then
// `sync()` (every wave past the K loop, the tile's pair rows in LDS), then
// the epilogue with the next tile's plan and first copies (`issue(part)`)
// issued before it and between its blocks: the copies' latency hides under
// the epilogue, and the epilogue's VALU work fills the time a wave waits
// for the memory pipeline to accept them.  (All copies after the epilogue
// measured slower: their latency is then exposed.)
// NB = the wave's 32-token blocks holding routed tokens (0..3).
template <int MODE, int NB, class Sync, class Issue>
__device__ __forceinline__ void xp_tile(const XCopies& c, const GArgs& g, uint8_t* smem, uint32_t ring,
                                        const XpTile& t, int wave, int lane, Sync&& sync, Issue&& issue) {
    const int wm = wave >> 2, wn = wave & 3;
    const int lr = lane & 31, h = lane >> 5;
    const int key = mx::swz_key128(lr);
    const int nsteps = g.Kp / 256;
    mx::v16f acc[3][2];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;

    for (int it = 0; it < nsteps; ++it) {
        // this wave's copies of step it have landed (the weights of step
        // it+1, issued last, may still be in flight) and its reads of step
        // it-1 are done; after the barrier every wave's
        if (it + 1 < nsteps) asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        const bool more_a = it + 1 < nsteps, more_w = it + 2 < nsteps;
        const uint8_t* wst = smem + ((it + 1) % 3) * X_WST;
        const uint8_t* ast = smem + X_ARING + (it & 1) * X_AST;
        const uint32_t anxt = ring + X_ARING + ((it + 1) & 1) * X_AST;
        const uint32_t wnxt = ring + (it % 3) * X_WST;   // step it+2: stage (it+3) % 3, step it-1's
        const uint8_t* la = ast + (32 * wm + lr) * X_ROWB;
        const uint8_t* lw = wst + (wn * 64 + lr) * X_ROWB;
        const uint8_t* lsa = ast + X_A + (32 * wm + lr) * 8;
        const uint8_t* lsw = wst + X_W + (wn * 64 + lr) * 8;
        uint32_t sa[3], sb[2];
#pragma unroll
        for (int i = 0; i < NB; ++i) sa[i] = scale_word(lsa + i * 64 * 8, h);
#pragma unroll
        for (int j = 0; j < 2; ++j) sb[j] = scale_word(lsw + j * 32 * 8, h);
        uint4 af[2][3], bf[2][2];
        auto load = [&](int ks, int r) {
            const int koff = ((2 * ks + h) ^ key) << 4;
#pragma unroll
            for (int i = 0; i < NB; ++i) af[r][i] = *reinterpret_cast<const uint4*>(la + koff + i * 64 * X_ROWB);
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[r][j] = *reinterpret_cast<const uint4*>(lw + koff + j * 32 * X_ROWB);
        };
        if (NB > 0) load(0, 0);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            __builtin_amdgcn_sched_barrier(0);
            if (ks < 2) {
                if (more_a) x8_issue_a(c, anxt, it + 1, ks, wave);
            } else if (more_w) {
                x8_issue_w(c, wnxt, it + 2, ks, wave);
            }
            if (NB > 0) {
                if (ks + 1 < 4) load(ks + 1, (ks + 1) & 1);
                const int r = ks & 1;
#pragma unroll
                for (int i = 0; i < NB; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (ks == 0) acc[i][j] = mfma32<0>(bf[r][j], af[r][i], acc[i][j], sb[j], sa[i]);
                        if (ks == 1) acc[i][j] = mfma32<1>(bf[r][j], af[r][i], acc[i][j], sb[j], sa[i]);
                        if (ks == 2) acc[i][j] = mfma32<2>(bf[r][j], af[r][i], acc[i][j], sb[j], sa[i]);
                        if (ks == 3) acc[i][j] = mfma32<3>(bf[r][j], af[r][i], acc[i][j], sb[j], sa[i]);
                    }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) mx::pin(acc[i][j]);
    sync();
    issue(0);
    xp_epilogue<MODE, NB>(acc, g, smem, t, wave, lane, issue);
}

// Epilogue of one wave's token blocks (NB of them) of tile t; issues parts 1
// and 2 of the next tile's first copies between its blocks.
template <int MODE, int NB, class Issue>
__device__ __forceinline__ void xp_epilogue(mx::v16f (&acc)[3][2], const GArgs& g, uint8_t* smem, const XpTile& t,
                                            int wave, int lane, Issue&& issue) {
    const int wm = wave >> 2, wn = wave & 3;
    const int lr = lane & 31, h = lane >> 5;
    if (NB == 0) {
        issue(1);
        issue(2);
        return;
    }
    if (MODE == MODE_DOWN) {
        // bf16(bf16(y) * score) through LDS, one 32-token block at a time in
        // the wave's own 32-row buffer of weight stage 0, so that a store
        // writes 8 whole 128-byte row segments; rows 136 bytes apart make
        // the 8-byte writes of 32 lanes (one row each) hit distinct banks
        uint8_t* tb = smem + wave * 32 * XP_TROW;
        const int* lp = reinterpret_cast<const int*>(smem + X_PP);
        const float* ls = reinterpret_cast<const float*>(smem + X_PP + 4 * X_BM);
        // lane: buffer row 8*st + lane/8 (tile row 64*i + 32*wm + 8*st +
        // lane/8), 16 bytes at column chunk lane%8
        const int ch = lane & 7;
        const int col = t.n0 + wn * 64 + 8 * ch;
        const int lim = col < g.Nw ? t.mrows - 32 * wm - (lane >> 3) : 0;   // tile rows < lim + 32*wm + lane/8 are routed
        const uint8_t* tr = tb + (lane >> 3) * XP_TROW + 16 * ch;
        const int* pr = lp + 32 * wm + (lane >> 3);
        uint16_t* yc = g.yd + col;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const float sc = ls[64 * i + 32 * wm + lr];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    uint32_t b[2];
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        const uint32_t y2 = mx::f32x2_to_bf16x2(acc[i][j][4 * q4 + 2 * r], acc[i][j][4 * q4 + 2 * r + 1]);
                        b[r] = mx::f32x2_to_bf16x2(__uint_as_float(y2 << 16) * sc, __uint_as_float(y2 & 0xFFFF0000u) * sc);
                    }
                    // element q of block j: column 32j + 8(q/4) + 4h + q%4
                    *reinterpret_cast<uint2*>(tb + lr * XP_TROW + (32 * j + 8 * q4 + 4 * h) * 2) = make_uint2(b[0], b[1]);
                }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int toff = 64 * i + 8 * st;   // tile row - (32*wm + lane/8)
                if (toff < lim) {
                    const uint4 v = *reinterpret_cast<const uint4*>(tr + 8 * st * XP_TROW);
                    *reinterpret_cast<uint4*>(yc + (int64_t)pr[toff] * g.Nw) = v;
                }
            }
            if (i < 2) issue(i + 1);
        }
        if (NB == 1) issue(2);
        return;
    }
    const int pp[2] = {0, 0};
    const float ss[2] = {0.0f, 0.0f};
    if (NB >= 2) {
        mx::v16f sub[2][2] = {{acc[0][0], acc[0][1]}, {acc[1][0], acc[1][1]}};
        tile_epilogue<MODE, 2>(sub, g, t.n0, t.off, t.mt, t.mrows, 32 * wm, wn, lr, h, pp, ss, 64);
        issue(1);
    }
    if (NB == 1 || NB == 3) {
        mx::v16f sub[2][2] = {{acc[NB - 1][0], acc[NB - 1][1]}, {acc[NB - 1][0], acc[NB - 1][1]}};
        tile_epilogue<MODE, 1>(sub, g, t.n0, t.off, t.mt, t.mrows, 64 * (NB - 1) + 32 * wm, wn, lr, h, pp, ss, 64);
        if (NB == 1) issue(1);
    }
    issue(2);
}

template <int MODE, class W>
__global__ __launch_bounds__(X_THREADS, 1) void grouped_gemm_xp_kernel(GArgs g, W w, int ntiles, int n_exp,
                                                                       int* __restrict__ qctr) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int grp = blockIdx.x & 7;
    const int kw = blockIdx.x >> 3;              // workgroup of the group
    const int per = gridDim.x >> 3;              // workgroups per group
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ring = __builtin_amdgcn_readfirstlane(mx::lds_addr(smem));
    int* ucum = reinterpret_cast<int*>(smem + XP_UCUM);
    int* ecnt = reinterpret_cast<int*>(smem + XP_ECNT);
    int* eoff = reinterpret_cast<int*>(smem + XP_EOFF);
    int* slot = reinterpret_cast<int*>(smem + XP_SLOT);
    const int nj = n_exp > grp ? (n_exp - grp + 7) / 8 : 0;
    if (nj == 0) return;
    for (int j = tid; j < nj; j += X_THREADS) {
        ecnt[j] = g.counts[grp + 8 * j];
        eoff[j] = g.offs[grp + 8 * j];
    }
    __syncthreads();
    if (wave == 0) {   // units below expert j: exclusive prefix, two experts per lane
        const int j0 = 2 * lane;
        const int u0 = j0 < nj ? (ecnt[j0] + X_BM - 1) / X_BM * ntiles : 0;
        const int u1 = j0 + 1 < nj ? (ecnt[j0 + 1] + X_BM - 1) / X_BM * ntiles : 0;
        int v = u0 + u1;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(v, d);
            if (lane >= d) v += o;
        }
        const int ex = v - u0 - u1;
        ucum[j0] = ex;
        ucum[j0 + 1] = ex + u0;
        if (lane == 63) ucum[128] = v;
    }
    __syncthreads();
    const int nunits = __builtin_amdgcn_readfirstlane(ucum[nj]);
    // units kw and kw + per are this workgroup's first two; the queue hands
    // out the rest, from 2 * per on
    if (kw >= nunits) return;
    const int nsteps = g.Kp / 256;
    XpTile t = xp_tile_of<MODE>(smem, grp, nj, ntiles, kw, lane);
    XCopies c;
    {
        int rw[4];
        x8_rows<MODE>(rw, g, t.off, t.mt, t.mrows, wave, lane);
        x8_plan_rows<MODE>(c, g, w, t.e, t.n0, t.mrows, rw, wave, lane);
    }
    xp_prologue(c, ring, nsteps, wave);
    int un1 = kw + per;                          // the next tile's unit (uniform)
    const int trow = wave * 64 + lane;
    for (;;) {
        // Issued now, used only after the K loop: the next tile's source
        // rows, the queue's unit for the tile after it, and the down tile's
        // pair indices and weights.  No loaded value is merged with a
        // default (a merge is a use, and the compiler's wait for it would
        // also wait for the copies in flight, which it does not count): the
        // atomic's result is read only by the lane that issued it, every
        // load is unconditional (clamped rows).  atomicInc, because the
        // compiler's wave aggregation of atomic adds uses the result at once.
        const bool more = un1 < nunits;
        XpTile tn = t;
        int rwn[4];
        if (more) {
            tn = xp_tile_of<MODE>(smem, grp, nj, ntiles, un1, lane);
            x8_rows<MODE>(rwn, g, tn.off, tn.mt, tn.mrows, wave, lane);
        }
        int uq;
        if (tid == 0) uq = (int)atomicInc(reinterpret_cast<unsigned*>(qctr + grp), 0xFFFFFFFFu);
        int rp = 0;
        float rs = 0.0f;
        if (MODE == MODE_DOWN) {
            const int r = t.off + t.mt + min(trow, t.mrows - 1);
            rp = g.pairs[r];
            rs = g.sscore[r];
        }
        XCopies cn = c;
        auto sync = [&]() {
            if (MODE == MODE_DOWN && trow < t.mrows) {
                reinterpret_cast<int*>(smem + X_PP)[trow] = rp;
                reinterpret_cast<float*>(smem + X_PP + 4 * X_BM)[trow] = rs;
            }
            if (tid == 0) *slot = uq;
            // every wave is past its last operand read of this tile (the
            // next tile's copies may overwrite the stages), the pair rows
            // and the queue's unit are in LDS
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        };
        auto issue = [&](int part) {
            if (more) {
                if (part == 0) x8_plan_rows<MODE>(cn, g, w, tn.e, tn.n0, tn.mrows, rwn, wave, lane);
                xp_prologue_part(cn, ring, nsteps, wave, part);
            }
        };
        // the wave's token blocks 2i + wm (i < nb) holding routed rows
        const int nb = min(((t.mrows + 31) / 32 - (wave >> 2) + 1) >> 1, 3);
        switch (nb) {
            case 3: xp_tile<MODE, 3>(c, g, smem, ring, t, wave, lane, sync, issue); break;
            case 2: xp_tile<MODE, 2>(c, g, smem, ring, t, wave, lane, sync, issue); break;
            case 1: xp_tile<MODE, 1>(c, g, smem, ring, t, wave, lane, sync, issue); break;
            default: xp_tile<MODE, 0>(c, g, smem, ring, t, wave, lane, sync, issue); break;
        }
        if (!more) break;
        un1 = 2 * per + __builtin_amdgcn_readfirstlane(*slot);
        t = tn;
        c = cn;
    }
}

// out[t, c] = bf16(sum_{k < topk, id valid} yd[t*topk + k, c]); 8 columns per thread
__global__ __launch_bounds__(256) void prefill_combine_kernel(const uint16_t* __restrict__ yd,
                                                              const int64_t* __restrict__ topi, int T, int topk,
                                                              int H, int n_exp, uint16_t* __restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int per_row = H >> 3;
    if (gid >= (int64_t)T * per_row) return;
    const int t = (int)(gid / per_row);
    const int c = (int)(gid - (int64_t)t * per_row) * 8;
    float s[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = 0.0f;
    for (int k = 0; k < topk; ++k) {
        const int64_t id = topi[(int64_t)t * topk + k];
        if (id < 0 || id >= n_exp) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(yd + ((int64_t)t * topk + k) * H + c);
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s[2 * i] += mx::bf16_to_f32((uint16_t)(wv[i] & 0xFFFFu));
            s[2 * i + 1] += mx::bf16_to_f32((uint16_t)(wv[i] >> 16));
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o[i] = (uint32_t)mx::f32_to_bf16_rne(s[2 * i]) | ((uint32_t)mx::f32_to_bf16_rne(s[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(out + (int64_t)t * H + c) = make_uint4(o[0], o[1], o[2], o[3]);
}

// ------------------------------------------------------------------ host
struct WsLayout {
    size_t counts, offs, pairs, sscore, hist, qctr, xq, xs, hq, hs, yd, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// CUs per XCD of the current device (its CU count / 8), cached per device:
// the persistent grouped GEMMs launch one workgroup per CU.
int cus_per_xcd() {
    static int cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 32;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
        cache[dev] = n / 8;
    }
    return cache[dev];
}

WsLayout ws_layout(int T, int topk, int n_exp, int H, int Mi) {
    const size_t P = (size_t)T * topk;
    WsLayout L;
    size_t o = 0;
    L.counts = o; o = align256(o + sizeof(int) * n_exp);
    L.offs = o;   o = align256(o + sizeof(int) * n_exp);
    L.pairs = o;  o = align256(o + sizeof(int) * P);
    L.sscore = o; o = align256(o + sizeof(float) * P);
    L.hist = o;   o = align256(o + sizeof(int) * ((P + kRtChunk - 1) / kRtChunk) * n_exp);
    L.qctr = o;   o = align256(o + sizeof(int) * 16);
    L.xq = o;     o = align256(o + (size_t)T * (H / 2));
    L.xs = o;     o = align256(o + (size_t)T * (H / 32));
    L.hq = o;     o = align256(o + P * (Mi / 2));
    L.hs = o;     o = align256(o + P * (Mi / 32));
    L.yd = o;     o = align256(o + P * H * sizeof(uint16_t));
    L.total = o;
    return L;
}

template <class W>
int run_prefill(const void* x, const int64_t* topi, const uint16_t* scores, W w, int n_exp, int T, int topk,
                int H, int Mi, void* out, void* workspace, size_t ws_bytes, hipStream_t st) {
    MXH_REQUIRE(x && topi && scores && out && workspace, "moe_prefill: null pointer");
    MXH_REQUIRE(T > 0 && topk > 0 && topk <= kMaxTopk, "moe_prefill: T=%d topk=%d (need T > 0, 0 < topk <= %d)",
                T, topk, kMaxTopk);
    MXH_REQUIRE(n_exp > 0 && n_exp <= kMaxExperts, "moe_prefill: n_experts=%d (1..%d)", n_exp, kMaxExperts);
    MXH_REQUIRE(H > 0 && H % 32 == 0 && Mi > 0 && Mi % 32 == 0,
                "moe_prefill: H=%d and Mi=%d must be positive multiples of 32", H, Mi);
    MXH_REQUIRE((int64_t)T * topk < (1ll << 31) / 2, "moe_prefill: T*topk too large");
    MXH_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)workspace & 255) == 0,
                "moe_prefill: x/out must be 16-byte and workspace 256-byte aligned");
    const WsLayout L = ws_layout(T, topk, n_exp, H, Mi);
    MXH_REQUIRE(ws_bytes >= L.total, "moe_prefill: workspace of %zu bytes < required %zu", ws_bytes, L.total);
    static bool attr_set[2][6] = {};
    constexpr int tw = std::is_same<W, TableW>::value ? 1 : 0;
    for (int m = 0; m < 6; ++m) {
        if (attr_set[tw][m]) continue;
        const void* fns[6] = {reinterpret_cast<const void*>(grouped_gemm_kernel<MODE_GATEUP, W>),
                              reinterpret_cast<const void*>(grouped_gemm_kernel<MODE_DOWN, W>),
                              reinterpret_cast<const void*>(grouped_gemm_dma_kernel<MODE_GATEUP, W>),
                              reinterpret_cast<const void*>(grouped_gemm_dma_kernel<MODE_DOWN, W>),
                              reinterpret_cast<const void*>(grouped_gemm_xp_kernel<MODE_GATEUP, W>),
                              reinterpret_cast<const void*>(grouped_gemm_xp_kernel<MODE_DOWN, W>)};
        const int bytes = m < 2 ? 2 * BUF_BYTES : m < 4 ? D_NST * D_STAGE : XP_LDS;
        hipError_t e = hipFuncSetAttribute(fns[m], hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        MXH_REQUIRE(e == hipSuccess, "moe_prefill: cannot reserve %d B of LDS: %s", bytes, hipGetErrorString(e));
        attr_set[tw][m] = true;
    }
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    int* counts = reinterpret_cast<int*>(ws + L.counts);
    int* offs = reinterpret_cast<int*>(ws + L.offs);
    int* pairs = reinterpret_cast<int*>(ws + L.pairs);
    const int P = T * topk;

    float* sscore = reinterpret_cast<float*>(ws + L.sscore);
    int* hist = reinterpret_cast<int*>(ws + L.hist);
    const int nchunk = (P + kRtChunk - 1) / kRtChunk;
    int* qctr = reinterpret_cast<int*>(ws + L.qctr);
    // x -> fp16 -> MXFP4 once per token (the reference quantizes each gathered
    // copy; the bytes are identical), in the same launch: quantize_rows_kernel's
    // layout (x is 16-byte aligned and H a multiple of 32, so the vector path)
    XQuant xqa{x, T, H, 2, 0, ws + L.xq, ws + L.xs};
    while ((1 << xqa.lt) < H / 8 && xqa.lt < 8) ++xqa.lt;
    xqa.gx = (T + (256 >> xqa.lt) - 1) / (256 >> xqa.lt);
    const int xq_gy = (H / 8 + (1 << xqa.lt) - 1) >> xqa.lt;
    hipLaunchKernelGGL(route_count_kernel, dim3(nchunk + xqa.gx * xq_gy), dim3(64 * kRtWaves), 0, st, topi, P, n_exp,
                       hist, qctr, nchunk, xqa);
    hipLaunchKernelGGL(route_scatter_kernel, dim3(nchunk), dim3(64 * kRtWaves), 0, st, topi, P, n_exp, hist, counts,
                       offs, pairs, scores, sscore);
    int rc = mxh::launch_status("moe_prefill route");
    if (rc != MXFP4_OK) return rc;

    GArgs g{};
    g.counts = counts;
    g.offs = offs;
    g.pairs = pairs;
    g.topk = topk;
    g.hq = ws + L.hq;
    g.hs = ws + L.hs;
    g.yd = reinterpret_cast<uint16_t*>(ws + L.yd);
    g.sscore = sscore;

    g.aq = ws + L.xq;
    g.as = ws + L.xs;
    g.Kp = H;
    g.Nw = Mi;
    g.a_rows = T;
    // the copy kernels address operands with 32-bit byte offsets
    const bool fit_gu = (int64_t)T * (H / 2) < (1ll << 32) && (int64_t)Mi * (H / 2) < (1ll << 32);
    const bool fit_dn = (int64_t)P * (Mi / 2) < (1ll << 32) && (int64_t)H * (Mi / 2) < (1ll << 32);
    const int xp_grid = 8 * cus_per_xcd();   // one persistent workgroup per CU
    if (H % 256 == 0 && fit_gu) {
        const int ntiles = (Mi + X_BN / 2 - 1) / (X_BN / 2);
        hipLaunchKernelGGL((grouped_gemm_xp_kernel<MODE_GATEUP, W>), dim3(xp_grid), dim3(X_THREADS), XP_LDS, st, g,
                           w, ntiles, n_exp, qctr);
    } else if (H % DK == 0 && fit_gu)
        hipLaunchKernelGGL((grouped_gemm_dma_kernel<MODE_GATEUP, W>), dim3((Mi + 63) / 64, n_exp), dim3(256),
                           D_NST * D_STAGE, st, g, w);
    else
        hipLaunchKernelGGL((grouped_gemm_kernel<MODE_GATEUP, W>), dim3((Mi + 63) / 64, n_exp), dim3(256),
                           2 * BUF_BYTES, st, g, w);
    rc = mxh::launch_status("moe_prefill gate/up");
    if (rc != MXFP4_OK) return rc;

    g.aq = ws + L.hq;
    g.as = ws + L.hs;
    g.Kp = Mi;
    g.Nw = H;
    g.a_rows = P;
    if (Mi % 256 == 0 && fit_dn) {
        const int ntiles = (H + X_BN - 1) / X_BN;
        hipLaunchKernelGGL((grouped_gemm_xp_kernel<MODE_DOWN, W>), dim3(xp_grid), dim3(X_THREADS), XP_LDS, st, g,
                           w, ntiles, n_exp, qctr + 8);
    } else if (Mi % DK == 0 && fit_dn)
        hipLaunchKernelGGL((grouped_gemm_dma_kernel<MODE_DOWN, W>), dim3((H + BN - 1) / BN, n_exp), dim3(256),
                           D_NST * D_STAGE, st, g, w);
    else
        hipLaunchKernelGGL((grouped_gemm_kernel<MODE_DOWN, W>), dim3((H + BN - 1) / BN, n_exp), dim3(256),
                           2 * BUF_BYTES, st, g, w);
    rc = mxh::launch_status("moe_prefill down");
    if (rc != MXFP4_OK) return rc;

    const int64_t threads = (int64_t)T * (H / 8);
    hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint16_t*>(ws + L.yd), topi, T, topk, H, n_exp,
                       static_cast<uint16_t*>(out));
    return mxh::launch_status("moe_prefill combine");
}

}  // namespace

extern "C" int mxfp4_moe_group(const int64_t* topi, int T, int topk, int n_experts, int* counts, int* offsets,
                               int* pairs, void* stream) {
    MXH_REQUIRE(topi && counts && offsets && pairs, "moe_group: null pointer");
    MXH_REQUIRE(T > 0 && topk > 0 && (int64_t)T * topk < (1ll << 30), "moe_group: T=%d topk=%d", T, topk);
    MXH_REQUIRE(n_experts > 0 && n_experts <= kMaxExperts, "moe_group: n_experts=%d (1..%d)", n_experts, kMaxExperts);
    hipLaunchKernelGGL(route_kernel, dim3((n_experts + kRouteEpw - 1) / kRouteEpw), dim3(64 * kRouteWaves), 0,
                       mxh::as_stream(stream), topi, T * topk, n_experts,
                       counts, offsets, pairs, nullptr, nullptr);
    return mxh::launch_status("moe_group");
}

extern "C" size_t mxfp4_moe_prefill_workspace_size(int T, int topk, int n_experts, int H, int Mi) {
    if (T <= 0 || topk <= 0 || n_experts <= 0 || H <= 0 || Mi <= 0) return 0;
    return ws_layout(T, topk, n_experts, H, Mi).total;
}

extern "C" int mxfp4_moe_prefill(const void* x, const int64_t* topi, const uint16_t* scores,
                                 const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                                 const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws,
                                 int n_experts, int T, int topk, int H, int Mi, void* out, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(gate_wp && gate_ws && up_wp && up_ws && down_wp && down_ws, "moe_prefill: null weight pointer");
    MXH_REQUIRE(((uintptr_t)gate_wp & 15) == 0 && ((uintptr_t)up_wp & 15) == 0 && ((uintptr_t)down_wp & 15) == 0,
                "moe_prefill: packed weights must be 16-byte aligned");
    StackedW w;
    w.wp[0] = gate_wp; w.ws[0] = gate_ws;
    w.wp[1] = up_wp;   w.ws[1] = up_ws;
    w.wp[2] = down_wp; w.ws[2] = down_ws;
    w.wp_stride[0] = w.wp_stride[1] = (int64_t)Mi * (H / 2);
    w.ws_stride[0] = w.ws_stride[1] = (int64_t)Mi * (H / 32);
    w.wp_stride[2] = (int64_t)H * (Mi / 2);
    w.ws_stride[2] = (int64_t)H * (Mi / 32);
    return run_prefill(x, topi, scores, w, n_experts, T, topk, H, Mi, out, workspace, workspace_bytes,
                       mxh::as_stream(stream));
}

extern "C" int mxfp4_moe_prefill_tab(const void* x, const int64_t* topi, const uint16_t* scores,
                                     const int64_t* expert_tab, int n_experts, int T, int topk, int H, int Mi,
                                     void* out, void* workspace, size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(expert_tab, "moe_prefill_tab: null expert table");
    TableW w{expert_tab};
    return run_prefill(x, topi, scores, w, n_experts, T, topk, H, Mi, out, workspace, workspace_bytes,
                       mxh::as_stream(stream));
}
