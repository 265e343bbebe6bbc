// moe_batch.hip -- the MoE block of a batched decode step (M <= 16 tokens,
// top-E routing) in two launches, for the forward_batch caller
// (runtime/model_runner_v2.py:265-289: prequant of the normed rows, the
// token-major tables, moe_gateup, moe_down, moe_combine).
//
//   batch_gateup_kernel  workgroup (32-row block rb of Mi, slot s): the slot
//                        that first names an expert owns it and serves every
//                        token routed to it (at most one slot per token), so
//                        each routed expert's gate/up rows stream from HBM
//                        once per step; 4 waves = gate/up x two 16-row tiles
//                        on v_mfma_scale_f32_16x16x128_f8f6f4 (A = the
//                        tokens' MXFP4 rows, B = the weight rows).  Epilogue:
//                        h = silu(g) * u in fp32 and its MXFP4 32-block (the
//                        32 rows are one block of down's K), written per slot
//                        -- moe_down's own activation quantization
//                        (src/ext/mxfp4_decode.cu:218-279), bit-exact to it
//                        given g and u.
//   batch_down_kernel    two workgroups per 16 output columns, each with
//                        every other distinct expert (slot order); 12 waves
//                        share out a workgroup's experts; per expert, its
//                        down rows for the columns times the h rows of its
//                        tokens, weighted by the routing weights
//                        (moe_combine, src/ext/mxfp4_decode.cu:285-299) into
//                        per-wave token sums in LDS; the 12 wave sums are
//                        added in a fixed order and the two workgroups' sums
//                        are added into y, which the gate/up launch clears
//                        (two addends onto zero: the same bits in either
//                        order).  (150 VGPRs: 3 waves per SIMD, so 12 waves
//                        fit one CU.)  No gu / yd round trip through HBM and
//                        no separate combine launch.
//   batch_down_lds_kernel  the same down workgroups and arithmetic with every
//                        slot's h row copied into LDS once per workgroup, the
//                        owners read from a table the gate/up launch writes,
//                        and two owners' weight rows in flight per wave (the
//                        launcher's choice whenever the h rows fit in LDS).
//
// The results match the drop-in chain up to fp32 summation order (the
// combine adds a token's experts grouped by wave instead of in slot order).
#include <mutex>

#include "lds_dma.h"
#include "mx_device.h"
#include "mx_host.h"

namespace {

constexpr int kMaxTok = 16;     // tokens per step: one MFMA row tile
constexpr int kMaxE = 8;        // slots per token (moe_combine's cap)
constexpr int kMaxSlots = kMaxTok * kMaxE;
constexpr int kSegB = 4;        // MFMA K-steps per prefetch segment (mx::seg_scales_issue covers 4)
constexpr int kDownWaves = 12;   // 3 waves per SIMD at 150 VGPRs

struct BatchArgs {
    const uint8_t* xq;   // (M, H/2) MXFP4 activation rows
    const uint8_t* xs;   // (M, H/32)
    const int32_t* ids;  // (M, E) expert ids, token-major slots
    const float* w;      // (M, E) routing weights
    const uint8_t* gwp;  // stacked experts: gate/up (n, Mi, H/2) + (n, Mi, H/32)
    const uint8_t* gws;
    const uint8_t* uwp;
    const uint8_t* uws;
    const uint8_t* dwp;  // down (n, H, Mi/2) + (n, H, Mi/32)
    const uint8_t* dws;
    int n_experts, M, E, H, Mi;
    uint8_t* hq;         // (S, Mi/2) MXFP4 h per slot
    uint8_t* hs;         // (S, Mi/32)
    float* y;            // (M, H) fp32 MoE output
    uint8_t* meta;       // per slot: owner flag (S bytes), member count (S), member slots (S x 16)
};

// Workspace: h rows, h scales, then the owner table the gate/up launch writes
// for the down launch, 16-byte aligned.
__host__ __device__ constexpr size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t meta_offset(int S, int Mi) { return align16((size_t)S * (Mi / 2) + (size_t)S * (Mi / 32)); }
__host__ __device__ constexpr size_t meta_bytes(int S) { return (size_t)S * (2 + kMaxTok); }

// One prefetch segment: weight (B) and activation (A) 16-byte blocks and
// their scale bytes for kSegB MFMA K-steps.
struct Seg {
    uint4 b[kSegB];
    mx::SegScales bs;
    uint4 a[kSegB];
    mx::SegScales as;
};

// Lane (row l%16, group q = l/16) takes 32-block 4*st + q at K-step st (64
// contiguous bytes per row and load instruction); rows past the A rows
// (tokens) or blocks past the row read zeros with scale code 127.
__device__ __forceinline__ void load_seg(Seg& sg, const uint8_t* wrow, const uint8_t* srow, const uint8_t* arow,
                                         const uint8_t* asrow, bool aok, int q, int st0, int steps, int nch) {
#pragma unroll
    for (int j = 0; j < kSegB; ++j) {
        const int c = 4 * (st0 + j) + q;
        const bool ok = (st0 + j < steps) && (c < nch);
        sg.b[j] = ok ? *reinterpret_cast<const uint4*>(wrow + c * 16) : make_uint4(0, 0, 0, 0);
        sg.a[j] = (ok && aok) ? *reinterpret_cast<const uint4*>(arow + c * 16) : make_uint4(0, 0, 0, 0);
    }
    mx::seg_scales_issue(sg.bs, srow, q, st0, nch);
    mx::seg_scales_issue(sg.as, asrow, q, st0, nch);   // asrow is a valid row even when !aok
}

__device__ __forceinline__ mx::v4f mma_seg(const Seg& sg, bool aok, int q, int st0, int steps, int nch, mx::v4f acc) {
#pragma unroll
    for (int j = 0; j < kSegB; ++j)
        if (st0 + j < steps)
            acc = mx::mfma16_fp4(sg.a[j], sg.b[j], acc, mx::seg_scale_at(sg.as, j, aok, q, st0, steps, nch),
                                 mx::seg_scale_at(sg.bs, j, true, q, st0, steps, nch));
    return acc;
}

// The whole K loop of one 16 x 16 tile, two segments in flight.
__device__ __forceinline__ mx::v4f kloop(const uint8_t* wrow, const uint8_t* srow, const uint8_t* arow,
                                         const uint8_t* asrow, bool aok, int q, int steps, int nch) {
    mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
    Seg s0, s1;
    load_seg(s0, wrow, srow, arow, asrow, aok, q, 0, steps, nch);
    for (int st = 0; st < steps; st += 2 * kSegB) {
        if (st + kSegB < steps) load_seg(s1, wrow, srow, arow, asrow, aok, q, st + kSegB, steps, nch);
        acc = mma_seg(s0, aok, q, st, steps, nch, acc);
        if (st + kSegB >= steps) break;
        if (st + 2 * kSegB < steps) load_seg(s0, wrow, srow, arow, asrow, aok, q, st + 2 * kSegB, steps, nch);
        acc = mma_seg(s1, aok, q, st + kSegB, steps, nch, acc);
    }
    return acc;
}

// Owners: slot j owns its expert when its id is valid and no earlier slot
// names the same id.  Every thread of the workgroup holds the ids in LDS; the
// first-occurrence test reads them as broadcast 16-byte words, so it costs S/4
// LDS reads per slot with no data-dependent exit.
__device__ __forceinline__ bool first_occurrence(const int* s_ids, int S, int j, int n_experts) {
    if (j >= S) return false;
    const int e = s_ids[j];
    bool own = e >= 0 && e < n_experts;
    for (int k0 = 0; k0 < S; k0 += 4) {
        const int4 v = *reinterpret_cast<const int4*>(s_ids + k0);
        own &= !((k0 < j && v.x == e) || (k0 + 1 < j && v.y == e) || (k0 + 2 < j && v.z == e) ||
                 (k0 + 3 < j && v.w == e));
    }
    return own;
}

// STAGED (H <= 2048): the member tokens' activation rows and every scale byte
// are copied into LDS (LDS DMA) and each wave has all of its K steps of
// weight rows in flight at once; otherwise two 4-step segments of A and B go
// through registers (kloop).  Both run the same MFMA chain, so h is the same.
constexpr int kGuMaxSteps = 16;   // K steps (H/128) of the staged path

__host__ __device__ constexpr int gu_arow(int H) { return H / 2 + 16; }   // LDS bytes per A row
__host__ __device__ constexpr int gu_sa_off(int H) { return kMaxTok * gu_arow(H); }
__host__ __device__ constexpr int gu_sb_off(int H) { return gu_sa_off(H) + (int)align16((size_t)kMaxTok * (H / 32)); }
__host__ __device__ constexpr int gu_lds_bytes(int H) { return gu_sb_off(H) + 4 * 16 * (H / 32); }

template <bool STAGED>
__global__ __launch_bounds__(256) void batch_gateup_kernel(BatchArgs a) {
    __shared__ int s_slot[kMaxTok];
    __shared__ int s_cnt, s_own;
    __shared__ float gu[2][kMaxTok][33];
    const int rb = blockIdx.x, s = blockIdx.y;
    const int S = a.M * a.E;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int e = a.ids[s];
    // the down launch adds two halves into y: the workgroups of slot 0 clear it
    if (s == 0) {
        const int n = a.M * a.H, per = (n + gridDim.x - 1) / gridDim.x;
        for (int i = rb * per + tid; i < min(n, (rb + 1) * per); i += 256) a.y[i] = 0.0f;
    }
    // ---- the first slot naming expert e owns it and gathers its tokens: all
    // S <= 128 ids in one round of loads (two per lane), then ballots
    if (wave == 0) {
        const int v0 = lane < S ? a.ids[lane] : -1;
        const int v1 = 64 + lane < S ? a.ids[64 + lane] : -1;
        const bool any = __ballot((lane < s && v0 == e) || (64 + lane < s && v1 == e)) != 0ull;
        const unsigned long long b0 = __ballot(lane >= s && lane < S && v0 == e);
        const unsigned long long b1 = __ballot(64 + lane >= s && 64 + lane < S && v1 == e);
        const unsigned long long below = (1ull << lane) - 1ull;
        if (!any) {
            const int p0 = __popcll(b0 & below), p1 = __popcll(b0) + __popcll(b1 & below);
            if (((b0 >> lane) & 1ull) && p0 < kMaxTok) s_slot[p0] = lane;
            if (((b1 >> lane) & 1ull) && p1 < kMaxTok) s_slot[p1] = 64 + lane;
        }
        if (lane == 0) {
            const int cnt = __popcll(b0) + __popcll(b1);
            s_own = any ? 0 : 1;
            s_cnt = cnt < kMaxTok ? cnt : kMaxTok;
        }
    }
    __syncthreads();
    const bool valid_e = e >= 0 && e < a.n_experts;   // other ids contribute h = 0
    // the owner table of the down launch: slot s owns a valid expert (first
    // slot naming it), its member count and member slots (token order)
    if (rb == 0 && wave == 0) {
        const int S_ = a.M * a.E;
        if (lane == 0) {
            a.meta[s] = (uint8_t)(s_own && valid_e ? 1 : 0);
            a.meta[S_ + s] = (uint8_t)(s_own ? s_cnt : 0);
        }
        if (s_own && lane < s_cnt) a.meta[2 * S_ + s * kMaxTok + lane] = (uint8_t)s_slot[lane];
    }
    if (!s_own) return;
    const int cnt = s_cnt;
    const int l16 = lane & 15, q = lane >> 4;
    const int H = a.H, Mi = a.Mi;
    const int proj = wave >> 1;
    const int row = rb * 32 + (wave & 1) * 16 + l16;
    const int64_t ee = valid_e ? e : 0;
    const uint8_t* wrow = (proj ? a.uwp : a.gwp) + (ee * Mi + row) * (int64_t)(H / 2);
    const uint8_t* srow = (proj ? a.uws : a.gws) + (ee * Mi + row) * (int64_t)(H / 32);
    const bool aok = valid_e && l16 < cnt;
    const int nch = H / 32;
    mx::v4f acc;
    if constexpr (STAGED) {
        extern __shared__ __align__(16) uint8_t dyn[];
        const int steps = nch / 4;
        const uint32_t lds0 = mx::lds_addr(dyn);
        // member rows of x (wave w: members w, w + 4, ...) at t * gu_arow(H)
        const mx::v4u rx = mx::buf_rsrc(a.xq, (int64_t)a.M * (H / 2));
        for (int t = wave; t < cnt; t += 4) {
            const int tk = s_slot[t] / a.E;
            for (int c = 0; c * 1024 < H / 2; ++c)
                if (c * 1024 + 16 * lane < H / 2)
                    mx::dma16(16u * lane, rx, (uint32_t)(tk * (H / 2) + c * 1024), lds0 + t * gu_arow(H) + c * 1024);
        }
        // their scales, H/32 bytes per member at t * H/32: 4 bytes a lane, 64 / (H/128) members a copy
        const int lpr = H / 128, rpc = 64 / lpr;
        const mx::v4u rxs = mx::buf_rsrc(a.xs, (int64_t)a.M * nch);
        for (int t0 = wave * rpc; t0 < cnt; t0 += 4 * rpc) {
            const int t = t0 + lane / lpr;
            if (t < cnt)
                mx::dma4((uint32_t)((s_slot[t] / a.E) * nch + 4 * (lane % lpr)), rxs, 0u, lds0 + gu_sa_off(H) + t0 * nch);
        }
        // this wave's 16 weight rows' scales (16 x H/32 contiguous bytes)
        const mx::v4u rbs = mx::buf_rsrc(srow - (int64_t)l16 * nch, 16 * nch);
        for (int c = 0; c * 1024 < 16 * nch; ++c)
            if (c * 1024 + 16 * lane < 16 * nch)
                mx::dma16(16u * lane, rbs, (uint32_t)(c * 1024), lds0 + gu_sb_off(H) + wave * 16 * nch + c * 1024);
        // every K step of the wave's weight rows in flight
        uint4 bq[kGuMaxSteps];
#pragma unroll
        for (int st = 0; st < kGuMaxSteps; ++st)
            if (st < steps) bq[st] = *reinterpret_cast<const uint4*>(wrow + 16 * (4 * st + q));
        // all of it has landed (the copies of every wave, at the barrier)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const uint8_t* al = dyn + l16 * gu_arow(H);
        const uint8_t* asl = dyn + gu_sa_off(H) + l16 * nch;
        const uint8_t* bsl = dyn + gu_sb_off(H) + wave * 16 * nch + l16 * nch;
        acc = (mx::v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < kGuMaxSteps; ++st) {
            if (st < steps) {
                const int c = 4 * st + q;
                const uint4 av = aok ? *reinterpret_cast<const uint4*>(al + 16 * c) : make_uint4(0, 0, 0, 0);
                const uint32_t sa = aok ? (uint32_t)asl[c] : 127u;
                acc = mx::mfma16_fp4(av, bq[st], acc, sa, (uint32_t)bsl[c]);
            }
        }
    } else {
        const int tok = aok ? s_slot[l16] / a.E : 0;
        const uint8_t* arow = a.xq + (int64_t)tok * (H / 2);
        const uint8_t* asrow = a.xs + (int64_t)tok * (H / 32);
        acc = kloop(wrow, srow, arow, asrow, aok, q, (nch + 3) / 4, nch);
    }
    mx::pin(acc);
    // D[4q + i][l16]: token 4q + i of the group, weight row l16 of the tile
#pragma unroll
    for (int i = 0; i < 4; ++i) gu[proj][4 * q + i][(wave & 1) * 16 + l16] = acc[i];
    __syncthreads();
    // ---- h = silu(g) * u and its MXFP4 block: thread = (token tt, rows 2j, 2j+1)
    const int tt = tid >> 4, j = tid & 15;
    float h0 = 0.0f, h1 = 0.0f;
    if (tt < cnt) {
        h0 = mx::silu_mul(gu[0][tt][2 * j], gu[1][tt][2 * j]);
        h1 = mx::silu_mul(gu[0][tt][2 * j + 1], gu[1][tt][2 * j + 1]);
    }
    float am = fmaxf(__builtin_fabsf(h0), __builtin_fabsf(h1));
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) am = fmaxf(am, __shfl_xor(am, o));
    const uint32_t code = mx::e8m0_code(am);
    const float inv = mx::e8m0_inv_scale(code);
    uint32_t byte = mx::e2m1_code(h0 * inv) | (mx::e2m1_code(h1 * inv) << 4);
    byte |= (uint32_t)__shfl_down((int)byte, 1) << 8;
    byte |= (uint32_t)__shfl_down((int)byte, 2) << 16;
    if (tt < cnt) {
        const int64_t slot = s_slot[tt];
        if ((j & 3) == 0) *reinterpret_cast<uint32_t*>(a.hq + slot * (Mi / 2) + rb * 16 + j) = byte;
        if (j == 0) a.hs[slot * (Mi / 32) + rb] = (uint8_t)code;
    }
}

// Two workgroups per column block, each with every other owner (owners k
// with k % 2 == half): a wave walks half as many experts.  Each adds its
// partial sums into y, which the gate/up launch cleared: y = (0 + p_a) + p_b,
// the same bits in either arrival order (fp32 addition commutes).
__global__ __launch_bounds__(64 * kDownWaves) void batch_down_kernel(BatchArgs a) {
    __shared__ __align__(16) int s_ids[kMaxSlots];
    __shared__ int s_owner[kMaxSlots];
    __shared__ int s_flag[kMaxSlots];
    __shared__ int s_nown;
    __shared__ float s_w[kMaxSlots];
    __shared__ int s_mem[kDownWaves][kMaxTok];
    __shared__ float ypart[kDownWaves][kMaxTok][17];
    const int cb = blockIdx.x >> 1, half = blockIdx.x & 1;
    const int S = a.M * a.E;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, q = lane >> 4;
    if (tid < kMaxSlots) {
        s_ids[tid] = tid < S ? a.ids[tid] : -1;
        s_w[tid] = tid < S ? a.w[tid] : 0.0f;   // routing weights: read once, not per owner after its MFMAs
    }
    for (int i = tid; i < kDownWaves * kMaxTok * 17; i += 64 * kDownWaves) (&ypart[0][0][0])[i] = 0.0f;
    __syncthreads();
    // owners: slots whose expert no earlier slot names (slot order)
    if (tid < S) s_flag[tid] = first_occurrence(s_ids, S, tid, a.n_experts) ? 1 : 0;
    __syncthreads();
    if (wave == 0) {
        int n = 0;
        for (int j0 = 0; j0 < S; j0 += 64) {
            const int j = j0 + lane;
            const bool f = j < S && s_flag[j];
            const unsigned long long b = __ballot(f);
            if (f) s_owner[n + __popcll(b & ((1ull << lane) - 1ull))] = j;
            n += __popcll(b);
        }
        if (lane == 0) s_nown = n;
    }
    __syncthreads();
    const int nown = s_nown;
    const int H = a.H, Mi = a.Mi;
    const int nch = Mi / 32, steps = (nch + 3) / 4;
    const int col = cb * 16 + l16;   // this lane's weight row of down = output column
    // wave w of half h: owners 2 w + h, 2 (w + kDownWaves) + h, ...
    for (int k = 2 * wave + half; k < nown; k += 2 * kDownWaves) {
        const int slot0 = s_owner[k];
        const int e = s_ids[slot0];
        // the owner's slots (one per token), in slot order
        int cnt = 0;
        for (int j0 = slot0; j0 < S; j0 += 64) {
            const int j = j0 + lane;
            const bool mm = j < S && s_ids[j] == e;
            const unsigned long long b = __ballot(mm);
            const int pos = cnt + __popcll(b & ((1ull << lane) - 1ull));
            if (mm && pos < kMaxTok) s_mem[wave][pos] = j;
            cnt += __popcll(b);
        }
        cnt = cnt < kMaxTok ? cnt : kMaxTok;
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the wave's s_mem writes are visible to its lanes
        __builtin_amdgcn_wave_barrier();
        const bool aok = l16 < cnt;
        const int mslot = aok ? s_mem[wave][l16] : 0;
        const uint8_t* wrow = a.dwp + ((int64_t)e * H + col) * (Mi / 2);
        const uint8_t* srow = a.dws + ((int64_t)e * H + col) * (Mi / 32);
        const uint8_t* arow = a.hq + (int64_t)mslot * (Mi / 2);
        const uint8_t* asrow = a.hs + (int64_t)mslot * (Mi / 32);
        mx::v4f acc = kloop(wrow, srow, arow, asrow, aok, q, steps, nch);
        // D[4q + i][l16]: member 4q + i, column l16; weighted into its token's sum
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * q + i;
            if (r < cnt) {
                const int sl = s_mem[wave][r];
                ypart[wave][sl / a.E][l16] = fmaf(s_w[sl], acc[i], ypart[wave][sl / a.E][l16]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();   // s_mem is rewritten by the next owner
    }
    __syncthreads();
    for (int i = tid; i < a.M * 16; i += 64 * kDownWaves) {
        const int m = i >> 4, c = i & 15;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kDownWaves; ++w) v += ypart[w][m][c];
        __hip_atomic_fetch_add(a.y + (int64_t)m * H + cb * 16 + c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The down launch with the h rows in LDS (when they fit): every slot's MXFP4
// h row and scales are copied into LDS once per workgroup (LDS DMA), the
// owners come from the table the gate/up launch wrote (no first-occurrence
// pass), and a wave issues the down rows of up to two of its owners before
// it waits, so both owners' weights are in flight at once.  Same workgroups,
// same arithmetic and the same y additions as batch_down_kernel, so the
// results are identical.
constexpr int kOwnPerRound = 2;   // owners whose weights a wave has in flight at once

struct DownLds {
    int hrow;        // LDS bytes per h row (Mi/2 + 16: rows land in different bank groups)
    int hs_off;      // h scales: S x Mi/32 bytes
    int bs_off;      // B scales: per wave and owner in flight, 16 rows x Mi/32 bytes
    int bytes;
};

__host__ __device__ inline DownLds down_lds_layout(int S, int Mi) {
    DownLds d;
    d.hrow = Mi / 2 + 16;
    d.hs_off = (int)align16((size_t)S * d.hrow);
    d.bs_off = d.hs_off + (int)align16((size_t)S * (Mi / 32));
    d.bytes = d.bs_off + kDownWaves * kOwnPerRound * 16 * (Mi / 32);
    return d;
}

// k-th set bit (k from 0) of the 128-bit mask (lo, hi); -1 if there is none
__device__ __forceinline__ int nth_set(uint64_t lo, uint64_t hi, int k) {
    const int nlo = __popcll(lo);
    uint64_t m = k < nlo ? lo : hi;
    int kk = k < nlo ? k : k - nlo;
    if (kk >= __popcll(m)) return -1;
    for (int i = 0; i < kk; ++i) m &= m - 1;
    return (k < nlo ? 0 : 64) + (int)__ffsll((long long)m) - 1;
}

// MS: K steps bound; OPR <= kOwnPerRound: owners per round (1 at MS = 16, where
// two owners' rows would not fit the registers of 3 waves per SIMD).
template <int MS, int OPR>
__global__ __launch_bounds__(64 * kDownWaves) void batch_down_lds_kernel(BatchArgs a) {
    extern __shared__ __align__(16) uint8_t dyn[];
    __shared__ float s_w[kMaxSlots];
    __shared__ int s_mem[kDownWaves][OPR][kMaxTok];
    __shared__ float ypart[kDownWaves][kMaxTok][17];
    const int cb = blockIdx.x >> 1, half = blockIdx.x & 1;
    const int S = a.M * a.E;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q = lane >> 4;
    const int H = a.H, Mi = a.Mi;
    const int kb = Mi / 32, steps = (kb + 3) / 4;
    const DownLds L = down_lds_layout(S, Mi);
    const uint32_t lds0 = mx::lds_addr(dyn);
    // ---- owners (slot order) from the gate/up launch's table: every wave holds the mask.
    // These loads are waited for before any LDS copy is issued: the compiler's waits do
    // not count the copies (inline asm), so a wait issued after them would wait for them.
    const uint8_t* own = a.meta;
    const uint8_t* mcnt = a.meta + S;
    const uint8_t* mslots = a.meta + 2 * S;
    const bool o0 = lane < S && own[lane] != 0, o1 = 64 + lane < S && own[64 + lane] != 0;
    const uint64_t mlo = __ballot(o0), mhi = __ballot(o1);
    const int nown = __popcll(mlo) + __popcll(mhi);
    if (tid < S) s_w[tid] = a.w[tid];
    for (int i = tid; i < kDownWaves * kMaxTok * 17; i += 64 * kDownWaves) (&ypart[0][0][0])[i] = 0.0f;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // ---- copies of every slot's h row and the h scales into LDS
    {
        const mx::v4u rh = mx::buf_rsrc(a.hq, (int64_t)S * (Mi / 2));
        for (int sl = wave; sl < S; sl += kDownWaves)
            if (lane < Mi / 32) mx::dma16(16u * lane, rh, (uint32_t)(sl * (Mi / 2)), lds0 + sl * L.hrow);
        const mx::v4u rhs = mx::buf_rsrc(a.hs, (int64_t)S * kb);
        for (int c = wave; c * 1024 < S * kb; c += kDownWaves)
            if (c * 1024 + 16 * lane < S * kb) mx::dma16(16u * lane, rhs, (uint32_t)(c * 1024), lds0 + L.hs_off + c * 1024);
    }
    bool first = true;
    // wave w of half h: owners 2 w + h, 2 (w + kDownWaves) + h, ... in rounds of OPR
    for (int k0 = 2 * wave + half; first || k0 < nown; k0 += 2 * kDownWaves * OPR) {
        int oslot[OPR], oe[OPR], ocnt[OPR], mv[OPR];
        uint4 bq[OPR][MS];
#pragma unroll
        for (int o = 0; o < OPR; ++o) {
            const int k = k0 + 2 * kDownWaves * o;
            oslot[o] = k < nown ? nth_set(mlo, mhi, k) : -1;
            const int sl = oslot[o] < 0 ? 0 : oslot[o];
            const int e = oslot[o] < 0 ? 0 : a.ids[sl];
            oe[o] = e;
            ocnt[o] = oslot[o] < 0 ? 0 : (int)mcnt[sl];
            mv[o] = lane < ocnt[o] ? (int)mslots[sl * kMaxTok + lane] : 0;   // written to LDS after the wait
            // the owner's down rows for the 16 columns (zero-extent for no owner) and their scales
            const uint8_t* wrow = a.dwp + ((int64_t)e * H + cb * 16) * (Mi / 2);
            const __amdgpu_buffer_rsrc_t rw =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wrow), (short)0, oslot[o] < 0 ? 0 : 16 * (Mi / 2), 0x00020000);
#pragma unroll
            for (int st = 0; st < MS; ++st) {
                const mx::v4u v = __builtin_amdgcn_raw_buffer_load_b128(rw, (uint32_t)(l16 * (Mi / 2) + 16 * min(4 * st + q, kb - 1)), 0, 0);
                bq[o][st] = make_uint4(v.x, v.y, v.z, v.w);
            }
            const mx::v4u rs = mx::buf_rsrc(a.dws + ((int64_t)e * H + cb * 16) * kb, oslot[o] < 0 ? 0 : 16 * kb);
            if (lane < kb) mx::dma16(16u * lane, rs, 0u, lds0 + L.bs_off + (wave * kOwnPerRound + o) * 16 * kb);
        }
        // everything this wave issued has landed; the first round also waits for every
        // wave's h copies (and the LDS clears above) at the barrier
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int o = 0; o < OPR; ++o)
            if (lane < kMaxTok) s_mem[wave][o][lane] = mv[o];
        if (first) __syncthreads();   // also orders the s_mem writes (wave-local) before their reads
        else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        first = false;
#pragma unroll
        for (int o = 0; o < OPR; ++o) {
            if (oslot[o] < 0) continue;
            const int cnt = ocnt[o];
            const bool aok = l16 < cnt;
            const int mslot = aok ? s_mem[wave][o][l16] : 0;
            const uint8_t* ha = dyn + mslot * L.hrow;
            const uint8_t* hsa = dyn + L.hs_off + mslot * kb;
            const uint8_t* bsa = dyn + L.bs_off + (wave * kOwnPerRound + o) * 16 * kb + l16 * kb;
            mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < MS; ++st) {
                if (st < steps) {
                    const int c = 4 * st + q;
                    const bool ok = c < kb;
                    const uint4 av = (aok && ok) ? *reinterpret_cast<const uint4*>(ha + 16 * c) : make_uint4(0, 0, 0, 0);
                    const uint32_t sa = (aok && ok) ? (uint32_t)hsa[c] : 127u;
                    const uint32_t sb = ok ? (uint32_t)bsa[c] : 127u;
                    acc = mx::mfma16_fp4(av, bq[o][st], acc, sa, sb);
                }
            }
            // D[4q + i][l16]: member 4q + i, column l16; weighted into its token's sum
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * q + i;
                if (r < cnt) {
                    const int sl = s_mem[wave][o][r];
                    ypart[wave][sl / a.E][l16] = fmaf(s_w[sl], acc[i], ypart[wave][sl / a.E][l16]);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): s_mem / ypart of this round done
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    for (int i = tid; i < a.M * 16; i += 64 * kDownWaves) {
        const int m = i >> 4, c = i & 15;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kDownWaves; ++w) v += ypart[w][m][c];
        __hip_atomic_fetch_add(a.y + (int64_t)m * H + cb * 16 + c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Scratch of mxfp4_moe_decode_batch_noalloc: the per-slot MXFP4 h and the
// owner table of up to kMaxSlots slots at Mi <= kNoAllocMaxMi, 141,568 bytes.
// One copy per GPU, held until the process ends; host code addresses it only
// through the pointer hipGetSymbolAddress returns for the current device.
constexpr int kNoAllocMaxMi = 2048;
constexpr size_t kScratchBytes = meta_offset(kMaxSlots, kNoAllocMaxMi) + meta_bytes(kMaxSlots);
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int scratch_on_current_device(void** out) {
    int dev = -1;
    MXH_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices,
                "moe_decode_batch_noalloc: no usable current device (%d)", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        MXH_REQUIRE(e == hipSuccess && p != nullptr, "moe_decode_batch_noalloc: hipGetSymbolAddress: %s",
                    hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MXFP4_OK;
}

int check_batch_args(const uint8_t* xq, const uint8_t* xs, const int32_t* ids, const float* w,
                     const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp, const uint8_t* up_ws,
                     const uint8_t* down_wp, const uint8_t* down_ws, int n_experts, int M, int E, int H, int Mi,
                     const float* y) {
    MXH_REQUIRE(xq && xs && ids && w && gate_wp && gate_ws && up_wp && up_ws && down_wp && down_ws && y,
                "moe_decode_batch: null pointer");
    MXH_REQUIRE(M >= 1 && M <= kMaxTok, "moe_decode_batch: M=%d outside 1..%d", M, kMaxTok);
    MXH_REQUIRE(E >= 1 && E <= kMaxE, "moe_decode_batch: E=%d outside 1..%d", E, kMaxE);
    MXH_REQUIRE(n_experts >= 1, "moe_decode_batch: n_experts=%d", n_experts);
    MXH_REQUIRE(H >= 128 && H % 128 == 0, "moe_decode_batch: H=%d must be a positive multiple of 128", H);
    MXH_REQUIRE(Mi >= 32 && Mi % 32 == 0, "moe_decode_batch: Mi=%d must be a positive multiple of 32", Mi);
    MXH_REQUIRE(((uintptr_t)xq & 15) == 0 && ((uintptr_t)gate_wp & 15) == 0 && ((uintptr_t)up_wp & 15) == 0 &&
                    ((uintptr_t)down_wp & 15) == 0,
                "moe_decode_batch: packed operands and the workspace must be 16-byte aligned");
    return MXFP4_OK;
}

// The down kernel with h in LDS when it fits (Mi <= 2048: a slot's h row is
// one LDS copy of <= 64 lanes; at most kDownLdsMax bytes of dynamic LDS).
constexpr int kDownLdsMax = 128 * 1024;

template <int MS, int OPR>
int launch_down_lds(const BatchArgs& a, int lds_bytes, hipStream_t st) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&batch_down_lds_kernel<MS, OPR>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kDownLdsMax);
    if (attr != hipSuccess) {
        mxh::set_error("moe_decode_batch (down): hipFuncSetAttribute: %s", hipGetErrorString(attr));
        return (int)attr;
    }
    hipLaunchKernelGGL((batch_down_lds_kernel<MS, OPR>), dim3(2 * (a.H / 16)), dim3(64 * kDownWaves), lds_bytes, st, a);
    return mxh::launch_status("moe_decode_batch (down)");
}

// The two launches; w8 holds h (S*(Mi/2) + S*(Mi/32) bytes) and the owner
// table at meta_offset(S, Mi), 16-byte aligned.
int launch_batch(const BatchArgs& a, hipStream_t st) {
    const int S = a.M * a.E;
    if (a.H <= 128 * kGuMaxSteps)
        hipLaunchKernelGGL(batch_gateup_kernel<true>, dim3(a.Mi / 32, S), dim3(256), gu_lds_bytes(a.H), st, a);
    else
        hipLaunchKernelGGL(batch_gateup_kernel<false>, dim3(a.Mi / 32, S), dim3(256), 0, st, a);
    const int rc = mxh::launch_status("moe_decode_batch (gate/up)");
    if (rc != MXFP4_OK) return rc;
    const DownLds L = down_lds_layout(S, a.Mi);
    const int steps = (a.Mi / 32 + 3) / 4;
    if (a.Mi <= 2048 && L.bytes <= kDownLdsMax)
        return steps <= 6 ? launch_down_lds<6, 2>(a, L.bytes, st) : launch_down_lds<16, 1>(a, L.bytes, st);
    hipLaunchKernelGGL(batch_down_kernel, dim3(2 * (a.H / 16)), dim3(64 * kDownWaves), 0, st, a);
    return mxh::launch_status("moe_decode_batch (down)");
}

}  // namespace

extern "C" size_t mxfp4_moe_decode_batch_workspace_size(int M, int E, int Mi) {
    if (M <= 0 || E <= 0 || Mi <= 0) return 0;
    return meta_offset(M * E, Mi) + meta_bytes(M * E);
}

extern "C" int mxfp4_moe_decode_batch(const uint8_t* xq, const uint8_t* xs, const int32_t* ids, const float* w,
                                      const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                                      const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws,
                                      int n_experts, int M, int E, int H, int Mi, float* y, void* ws,
                                      size_t ws_bytes, void* stream) {
    const int rc = check_batch_args(xq, xs, ids, w, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, M,
                                    E, H, Mi, y);
    if (rc != MXFP4_OK) return rc;
    MXH_REQUIRE(ws, "moe_decode_batch: null pointer");
    MXH_REQUIRE(ws_bytes >= mxfp4_moe_decode_batch_workspace_size(M, E, Mi),
                "moe_decode_batch: workspace of %zu bytes, %zu needed", ws_bytes,
                mxfp4_moe_decode_batch_workspace_size(M, E, Mi));
    MXH_REQUIRE(((uintptr_t)ws & 15) == 0, "moe_decode_batch: packed operands and the workspace must be 16-byte aligned");
    const int S = M * E;
    uint8_t* w8 = static_cast<uint8_t*>(ws);
    const BatchArgs a{xq, xs, ids, w, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, M, E, H, Mi,
                      w8, w8 + (size_t)S * (Mi / 2), y, w8 + meta_offset(S, Mi)};
    return launch_batch(a, mxh::as_stream(stream));
}

extern "C" int mxfp4_moe_decode_batch_noalloc(const uint8_t* xq, const uint8_t* xs, const int32_t* ids,
                                              const float* w, const uint8_t* gate_wp, const uint8_t* gate_ws,
                                              const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                                              const uint8_t* down_ws, int n_experts, int M, int E, int H, int Mi,
                                              float* y, void* stream) {
    const int rc = check_batch_args(xq, xs, ids, w, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, M,
                                    E, H, Mi, y);
    if (rc != MXFP4_OK) return rc;
    MXH_REQUIRE(Mi <= kNoAllocMaxMi, "moe_decode_batch_noalloc: Mi=%d exceeds the %d of its fixed scratch", Mi,
                kNoAllocMaxMi);
    MXH_REQUIRE(mxfp4_moe_decode_batch_workspace_size(M, E, Mi) <= kScratchBytes,
                "moe_decode_batch_noalloc: %zu bytes of h exceed the %zu-byte scratch",
                mxfp4_moe_decode_batch_workspace_size(M, E, Mi), kScratchBytes);
    void* sp = nullptr;
    const int rs = scratch_on_current_device(&sp);
    if (rs != MXFP4_OK) return rs;
    // Every h row and owner-table entry the down kernel reads is written by the
    // gate/up kernel of the same call, so nothing in the scratch has to start
    // at zero.
    const int S = M * E;
    uint8_t* w8 = static_cast<uint8_t*>(sp);
    const BatchArgs a{xq, xs, ids, w, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, M, E, H, Mi,
                      w8, w8 + (size_t)S * (Mi / 2), y, w8 + meta_offset(S, Mi)};
    return launch_batch(a, mxh::as_stream(stream));
}
