// gemv.hip -- grouped small-M block-scaled MFMA GEMV for gfx950.
//
// Serves the reference's decode operators on token-major pointer tables:
//   moe_gateup  (src/ext/mxfp4_decode.cu:177-212)  A = pre-quantized MXFP4 rows
//   moe_down    (src/ext/mxfp4_decode.cu:218-279)  A = MXFP4(silu(g)*u), built in LDS
//   lin_pq, M <= 16 rows (src/ext/mxfp4_decode.cu:135-170)
// and the weighted combine (src/ext/mxfp4_decode.cu:285-299).
//
// Design (MI355X-first rather than a translation of the sm_120a kernels):
// * One v_mfma_scale_f32_16x16x128_f8f6f4 consumes packed E2M1 + E8M0 for 16
//   weight rows x 128 K straight from registers: no nibble unpacking, no
//   dequant VALU work.  The activation rows (tokens) form the A operand, so a
//   weight row is read once for every token routed to it.
// * Table entries whose weight pointers are equal are grouped inside the
//   kernel (first occurrence owns the group, others exit): at M=9 speculative
//   verify an expert shared by several tokens is streamed from HBM once,
//   where the reference re-reads it per token.
// * Each lane loads 16 bytes (one 32-block) per MFMA step; at step s lane
//   group g = l/16 takes block 4s + g, so the four lanes of a row read 64
//   contiguous bytes per load instruction (a block permutation is free
//   because A and B lanes pair on the same K set).  Weight loads for a K
//   segment are issued before the MFMAs of the previous segment (software
//   prefetch).
// * The pointer tables travel by value in the kernel arguments, replacing the
//   reference's host-blocking H2D table copy (src/ext/mxfp4_decode_binding.cpp:58).
#include "mx_device.h"
#include "mx_host.h"

namespace {

constexpr int kMaxT = MXFP4_MAX_TABLE;
constexpr int kSeg = 4;  // MFMA K-steps (512 K) per prefetch segment

// A host table also carries its grouping, worked out on the host (the
// pointers are there already): info[t] = n | (f << 8), n entries share entry
// t's weights when t is the first of them (n = 0 otherwise), listed at
// mem[f ..].  The kernel then starts on its weights after one scalar load
// instead of a scan of the table (a dependent memory round trip).
struct HostTable {
    static constexpr bool kGrouped = true;
    const uint8_t* wp[kMaxT];
    const uint8_t* ws[kMaxT];
    uint32_t info[kMaxT];
    uint8_t mem[kMaxT];
    __device__ __forceinline__ const uint8_t* w(int i) const { return wp[i]; }
    __device__ __forceinline__ const uint8_t* s(int i) const { return ws[i]; }
};
struct DevTable {
    static constexpr bool kGrouped = false;
    const int64_t* wp;
    const int64_t* ws;
    __device__ __forceinline__ const uint8_t* w(int i) const { return reinterpret_cast<const uint8_t*>(wp[i]); }
    __device__ __forceinline__ const uint8_t* s(int i) const { return reinterpret_cast<const uint8_t*>(ws[i]); }
};

enum { MAP_PLAIN = 0, MAP_GATEUP = 1 };
enum { A_FP4 = 0, A_SILU = 1 };

struct GemvArgs {
    int T;     // entries in this launch
    int t0;    // global table index of local entry 0
    int E;     // slots per token (token-major mapping)
    int map;   // MAP_*
    int N;     // weight rows
    int K;     // logical K (A_SILU: gu row stride is 2K)
    int Kp;    // padded K of weights and activations
    const uint8_t* aq;  // A_FP4: (rows, Kp/2)
    const uint8_t* as;  // A_FP4: (rows, Kp/32)
    const float* gu;    // A_SILU: (rows, 2K)
    float* out;
    int64_t ld_out;
    int ncb;   // A_SILU: 64-column blocks per workgroup (one h tile build for all of them); 0 = 1
};

struct EntryMap {
    int src, dst, col;
};

__device__ __forceinline__ EntryMap map_entry(const GemvArgs& a, int tg) {
    EntryMap r;
    if (a.map == MAP_GATEUP) {
        // t = m*2E + proj*E + e  (src/ext/mxfp4_decode.cu:187-195)
        const int m = tg / (2 * a.E);
        const int rem = tg - m * 2 * a.E;
        const int proj = rem / a.E;
        const int e = rem - proj * a.E;
        r.src = m;
        r.dst = m * a.E + e;
        r.col = proj * a.N;
    } else {
        r.src = tg;
        r.dst = tg;
        r.col = 0;
    }
    return r;
}

// One prefetch segment of kSeg MFMA K-steps: weight (B) data + scales, and
// for A_FP4 the activation (A) data + scales.  Separate named buffers keep
// all register indices static.
struct SegBuf {
    uint4 b[kSeg];
    mx::SegScales bs;
    uint4 a[kSeg];
    mx::SegScales as;
};

struct SegCtx {
    const uint8_t* wrow;   // this lane's weight row
    const uint8_t* srow;   // its scale row
    const uint8_t* arow;   // A_FP4: activation row
    const uint8_t* asrow;  // A_FP4: activation scale row
    const uint8_t* lq;     // A_SILU: LDS row of quantized h
    const uint8_t* lsc;    // A_SILU: LDS scale row
    int g, steps, nch;   // lane group (block 4s + g at step s), steps, 32-blocks per row
    bool arow_ok;
};

template <int AMODE>
__device__ __forceinline__ void load_seg(SegBuf& sb, const SegCtx& cx, int s0) {
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
        const int s = s0 + j;
        const int c = 4 * s + cx.g;
        const bool ok = (s < cx.steps) && (c < cx.nch);
        sb.b[j] = ok ? *reinterpret_cast<const uint4*>(cx.wrow + c * 16) : make_uint4(0, 0, 0, 0);
        if (AMODE == A_FP4) {
            const bool aok = ok && cx.arow_ok;
            sb.a[j] = aok ? *reinterpret_cast<const uint4*>(cx.arow + c * 16) : make_uint4(0, 0, 0, 0);
        }
    }
    static_assert(kSeg == 4, "mx::seg_scales_issue covers 4 K-steps");
    mx::seg_scales_issue(sb.bs, cx.srow, cx.g, s0, cx.nch);
    if (AMODE == A_FP4) mx::seg_scales_issue(sb.as, cx.asrow, cx.g, s0, cx.nch);   // asrow is valid even when !arow_ok
}

template <int AMODE>
__device__ __forceinline__ mx::v4f compute_seg(const SegBuf& sb, const SegCtx& cx, int s0, mx::v4f acc) {
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
        const int s = s0 + j;
        if (s < cx.steps) {
            uint4 aq;
            uint32_t asc;
            if (AMODE == A_FP4) {
                aq = sb.a[j];
                asc = mx::seg_scale_at(sb.as, j, cx.arow_ok, cx.g, s0, cx.steps, cx.nch);
            } else {
                // rows past the group (arow_ok false) are zero: their LDS rows are not built
                const int c = 4 * s + cx.g;
                const bool ok = c < cx.nch && cx.arow_ok;
                aq = ok ? *reinterpret_cast<const uint4*>(cx.lq + c * 16) : make_uint4(0, 0, 0, 0);
                asc = ok ? (uint32_t)cx.lsc[c] : 127u;
            }
            acc = mx::mfma16_fp4(aq, sb.b[j], acc, asc, mx::seg_scale_at(sb.bs, j, true, cx.g, s0, cx.steps, cx.nch));
        }
    }
    return acc;
}

// NW row tiles of 16 weight rows per workgroup, each split over S K-parts
// (one wave per tile and part; the S partial sums meet in LDS in part order).
// NW = 1 spreads a small-N launch over more workgroups and S > 1 puts a
// row tile's bytes in flight at once (A_FP4 only), so more CUs stream at once.
// MB (A_SILU, one K segment per part): a.ncb column blocks per workgroup.
template <class Tab, int AMODE, int NW, int S, bool MB = false>
__global__ __launch_bounds__(64 * NW * S) void grouped_gemv_kernel(Tab tab, GemvArgs a) {
    extern __shared__ __align__(16) uint8_t s_dyn[];  // A_SILU: 16 rows of quantized h
    __shared__ int s_rows[kMaxT];
    __shared__ int s_cnt, s_first;
    __shared__ mx::v4f s_red[S > 1 ? S - 1 : 1][NW][64];

    const int t = blockIdx.y;
    if (t >= a.T) return;
    const int lane = threadIdx.x & 63;
    const int wave = (threadIdx.x >> 6) % NW;     // row tile
    const int part = (threadIdx.x >> 6) / NW;     // K part
    const uint8_t* wp = tab.w(t);
    const uint8_t* ws = tab.s(t);

    // ---- grouping: the first entry with this weight owns all of its rows
    if constexpr (Tab::kGrouped) {
        const uint32_t info = tab.info[t];
        const int n = (int)(info & 0xFFu);
        if (n == 0) return;   // a later entry of a group: its owner serves it
        if ((int)threadIdx.x < n) s_rows[threadIdx.x] = n == 1 ? t : tab.mem[(info >> 8) + threadIdx.x];
        if (threadIdx.x == 0) {
            s_first = 1;
            s_cnt = n;
        }
    } else if (threadIdx.x < 64) {
        bool dup = false;
        for (int j = lane; j < t; j += 64) dup |= (tab.w(j) == wp) && (tab.s(j) == ws);
        const bool any = __ballot(dup) != 0ull;
        int cnt = 0;
        if (!any) {
            for (int j0 = t; j0 < a.T; j0 += 64) {
                const int j = j0 + lane;
                const bool m = (j < a.T) && (tab.w(j) == wp) && (tab.s(j) == ws);
                const unsigned long long b = __ballot(m);
                if (m) s_rows[cnt + __popcll(b & ((1ull << lane) - 1ull))] = j;
                cnt += __popcll(b);
            }
        }
        if (lane == 0) {
            s_first = any ? 0 : 1;
            s_cnt = cnt;
        }
    }
    __syncthreads();
    if (!s_first) return;
    const int cnt = s_cnt;

    const int nch = a.Kp >> 5;            // 32-blocks per row
    const int steps = (nch + 3) >> 2;     // MFMA K-steps; lane group g takes blocks g, g + 4, ...
    const int r = lane & 15;
    const int g = lane >> 4;
    // column blocks of 16 * NW weight rows: a workgroup takes ncb of them
    // (A_SILU with one K segment per part only, otherwise 1)
    const int ncb = MB ? a.ncb : 1;
    auto blk_n0 = [&](int cbk) { return (blockIdx.x * ncb + cbk) * (16 * NW) + wave * 16; };
    const int n0 = blk_n0(0);
    const int nrow = min(n0 + r, a.N - 1);
    const uint8_t* wrow = wp + (int64_t)nrow * (a.Kp >> 1);
    const uint8_t* srow = ws + (int64_t)nrow * nch;

    uint8_t* sq = s_dyn;                              // [16][Kp/2]
    uint8_t* ssc = s_dyn + 16 * (a.Kp >> 1);          // [16][nch]

    // this wave's K part: MFMA K-steps [sb, se), blocks from 4*sb on
    const int spw = (steps + S - 1) / S;
    const int sb = min(steps, part * spw), se = min(steps, sb + spw);
    const int64_t boff = 4 * (int64_t)sb;
    for (int rt = 0; rt < cnt; rt += 16) {
        // A-operand source row of this lane (row r of the tile)
        const bool arow_ok = (rt + r) < cnt;
        int asrc = 0;
        if (AMODE == A_FP4 && arow_ok) asrc = map_entry(a, a.t0 + s_rows[rt + r]).src;
        const uint8_t* arow = a.aq + (int64_t)asrc * (a.Kp >> 1);
        const uint8_t* asrow = a.as + (int64_t)asrc * nch;
        const SegCtx cx{wrow + boff * 16, srow + boff, arow + boff * 16, asrow + boff,
                        sq + r * (a.Kp >> 1) + boff * 16, ssc + r * nch + boff,
                        g, se - sb, nch - (int)boff, arow_ok};
        SegBuf s0buf, s1buf;
        // A_SILU: the thread's first 8 g / u values are loaded before the
        // weights (loads complete in issue order: loaded after them, h would
        // wait for the weight segment too)
        const int upr = a.Kp >> 3;
        const int nbr = min(16, cnt - rt);
        float pg[8] = {}, pu[8] = {};
        if (AMODE == A_SILU && (int)threadIdx.x < nbr * upr) {
            const int u = threadIdx.x;
            const int rr = u / upr;
            const int k0 = (u - rr * upr) * 8;
            const EntryMap em = map_entry(a, a.t0 + s_rows[rt + rr]);
            const float* grow = a.gu + (int64_t)em.src * 2 * a.K;
            if ((a.K & 7) == 0 && k0 + 8 <= a.K && (((uintptr_t)a.gu) & 15) == 0) {
                // 16-byte loads: g and u of the thread's 8 values (rows of 2K floats, K % 8 == 0)
                const float4 g0 = *reinterpret_cast<const float4*>(grow + k0);
                const float4 g1 = *reinterpret_cast<const float4*>(grow + k0 + 4);
                const float4 u0 = *reinterpret_cast<const float4*>(grow + a.K + k0);
                const float4 u1 = *reinterpret_cast<const float4*>(grow + a.K + k0 + 4);
                pg[0] = g0.x; pg[1] = g0.y; pg[2] = g0.z; pg[3] = g0.w;
                pg[4] = g1.x; pg[5] = g1.y; pg[6] = g1.z; pg[7] = g1.w;
                pu[0] = u0.x; pu[1] = u0.y; pu[2] = u0.z; pu[3] = u0.w;
                pu[4] = u1.x; pu[5] = u1.y; pu[6] = u1.z; pu[7] = u1.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) {   // clamped: every load issued before any is used
                    const int k = min(k0 + i, a.K - 1);
                    pg[i] = grow[k];
                    pu[i] = grow[a.K + k];
                }
            }
        }
        if (sb < se) load_seg<AMODE>(s0buf, cx, 0);   // the weights stream while h is built
        if (AMODE == A_SILU) {
            // Build the group's rows of the 16-row A tile: h = silu(g)*u (fp32)
            // quantized per 32-block with the bit-exact rule (rows past the
            // group are read as zeros by compute_seg, so they are not built).
            for (int u = threadIdx.x; u < nbr * upr; u += 64 * NW * S) {   // quads stay together
                const int rr = u / upr;
                const int uu = u - rr * upr;
                const int k0 = uu * 8;
                float h[8];
                if (u == (int)threadIdx.x) {   // the values loaded above
#pragma unroll
                    for (int i = 0; i < 8; ++i) h[i] = (k0 + i < a.K) ? mx::silu_mul(pg[i], pu[i]) : 0.0f;
                } else {
                    const EntryMap em = map_entry(a, a.t0 + s_rows[rt + rr]);
                    const float* grow = a.gu + (int64_t)em.src * 2 * a.K;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int k = k0 + i;
                        h[i] = (k < a.K) ? mx::silu_mul(grow[k], grow[a.K + k]) : 0.0f;
                    }
                }
                float am = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) am = fmaxf(am, __builtin_fabsf(h[i]));
                am = fmaxf(am, __shfl_xor(am, 1));
                am = fmaxf(am, __shfl_xor(am, 2));
                const uint32_t code = mx::e8m0_code(am);
                *reinterpret_cast<uint32_t*>(sq + rr * (a.Kp >> 1) + uu * 4) =
                    mx::e2m1_pack8(h, mx::e8m0_inv_scale(code));
                if ((uu & 3) == 0) ssc[rr * nch + (uu >> 2)] = (uint8_t)code;
            }
            __syncthreads();
        }

        // the S partial sums in part order (parts 1.. hand theirs to part 0),
        // then D[4*(l/16)+i][l%16] (token row, weight row) of column block cbk
        auto finish = [&](mx::v4f acc, int cbk) {
            mx::pin(acc);
            if constexpr (S > 1) {
                if (part > 0) s_red[part - 1][wave][lane] = acc;
                __syncthreads();
                if (part == 0) {
#pragma unroll
                    for (int p = 1; p < S; ++p) {
                        const mx::v4f o = s_red[p - 1][wave][lane];
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[i] += o[i];
                    }
                }
            }
            const int col = blk_n0(cbk) + r;
            if (part == 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int rr = 4 * g + i;
                    if (rt + rr < cnt && col < a.N) {
                        const EntryMap em = map_entry(a, a.t0 + s_rows[rt + rr]);
                        a.out[(int64_t)em.dst * a.ld_out + em.col + col] = acc[i];
                    }
                }
            }
            if constexpr (S > 1) __syncthreads();   // s_red is reused by the next block
        };
        if constexpr (!MB) {
            mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
            if (sb < se) {
                for (int s0 = 0; s0 < cx.steps; s0 += 2 * kSeg) {
                    if (s0 + kSeg < cx.steps) load_seg<AMODE>(s1buf, cx, s0 + kSeg);
                    acc = compute_seg<AMODE>(s0buf, cx, s0, acc);
                    if (s0 + kSeg >= cx.steps) break;
                    if (s0 + 2 * kSeg < cx.steps) load_seg<AMODE>(s0buf, cx, s0 + 2 * kSeg);
                    acc = compute_seg<AMODE>(s1buf, cx, s0 + kSeg, acc);
                }
            }
            finish(acc, 0);
        } else {
            // one K segment per part: block cbk's weights sit in s0buf (even cbk)
            // or s1buf (odd), and the next block's are issued before the MFMAs
            auto blk_ctx = [&](int cbk) {
                const int nr = min(blk_n0(cbk) + r, a.N - 1);
                SegCtx c = cx;
                c.wrow = wp + (int64_t)nr * (a.Kp >> 1) + boff * 16;
                c.srow = ws + (int64_t)nr * nch + boff;
                return c;
            };
            for (int cbk = 0; cbk < ncb; cbk += 2) {
                if (cbk + 1 < ncb && sb < se) load_seg<AMODE>(s1buf, blk_ctx(cbk + 1), 0);
                mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
                if (sb < se) acc = compute_seg<AMODE>(s0buf, cx, 0, acc);
                finish(acc, cbk);
                if (cbk + 1 >= ncb) break;
                if (cbk + 2 < ncb && sb < se) load_seg<AMODE>(s0buf, blk_ctx(cbk + 2), 0);
                acc = mx::v4f{0.f, 0.f, 0.f, 0.f};
                if (sb < se) acc = compute_seg<AMODE>(s1buf, cx, 0, acc);
                finish(acc, cbk + 1);
            }
        }
        if (AMODE == A_SILU || S > 1) __syncthreads();  // LDS reused by the next row tile
    }
}

// Dense y (M, N) = A (M, Kp) W (N, Kp)^T for M <= 16 (lin_pq at decode
// sizes).  A workgroup holds R row tiles of 16 weight rows x S K-parts, one
// wave each: wave w takes row tile w % R and the MFMA K-steps [p*spw,
// (p+1)*spw) of part p = w / R.  Splitting K gives a small-N projection (the
// router's 128 rows, o_proj's 2048) enough waves to have all of its bytes in
// flight at once; the S partial sums meet in LDS in a fixed order.
template <int R, int S>
__global__ __launch_bounds__(64 * R * S) void lin_small_kernel(const uint8_t* __restrict__ aq,
                                                               const uint8_t* __restrict__ as,
                                                               const uint8_t* __restrict__ wp,
                                                               const uint8_t* __restrict__ ws, float* __restrict__ y,
                                                               int M, int N, int Kp, int spw) {
    __shared__ mx::v4f red[S > 1 ? S : 1][R][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rt = wave % R, part = wave / R;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int n0 = (blockIdx.x * R + rt) * 16;
    const int nch = Kp >> 5;
    const int steps = (nch + 3) >> 2;
    const int sb = part * spw;
    const int se = min(steps, sb + spw);
    mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (n0 < N && sb < se) {
        // the part's blocks start at 4 * sb: shift the row pointers there
        const int nrow = min(n0 + r, N - 1);
        const int arow_i = min(r, M - 1);
        const int64_t boff = 4 * (int64_t)sb;
        const SegCtx cx{wp + (int64_t)nrow * (Kp >> 1) + boff * 16, ws + (int64_t)nrow * nch + boff,
                        aq + (int64_t)arow_i * (Kp >> 1) + boff * 16, as + (int64_t)arow_i * nch + boff,
                        nullptr, nullptr, g, se - sb, nch - (int)boff, r < M};
        SegBuf s0buf, s1buf;
        load_seg<A_FP4>(s0buf, cx, 0);
        for (int s0 = 0; s0 < cx.steps; s0 += 2 * kSeg) {
            if (s0 + kSeg < cx.steps) load_seg<A_FP4>(s1buf, cx, s0 + kSeg);
            acc = compute_seg<A_FP4>(s0buf, cx, s0, acc);
            if (s0 + kSeg >= cx.steps) break;
            if (s0 + 2 * kSeg < cx.steps) load_seg<A_FP4>(s0buf, cx, s0 + 2 * kSeg);
            acc = compute_seg<A_FP4>(s1buf, cx, s0 + kSeg, acc);
        }
    }
    if constexpr (S > 1) {
        red[part][rt][lane] = acc;
        __syncthreads();
        if (part != 0) return;
#pragma unroll
        for (int p = 1; p < S; ++p) {
            const mx::v4f o = red[p][rt][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += o[i];
        }
    }
    // D[4*(l/16)+i][l%16]: token row, weight row
    const int col = n0 + r;
    if (col >= N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * g + i;
        if (m < M) y[(int64_t)m * N + col] = acc[i];
    }
}

// ---------------------------------------------------------------- RMSNorm -> lin_pq
// The decode step's "x = x + bf16(o); h = rms_norm(x) -> MXFP4; y = lin_pq(h)"
// (runtime/model_runner_v2.py:185-187 and :208 + :147-152; RMSNorm
// runtime/model_runner.py:20-25) in one launch for H = 2048 and M <= 16 rows.
// Every workgroup normalises the rows itself (threads 0..255, 8 elements a
// thread, the arithmetic of mxfp4_rmsnorm_quant) into LDS and runs the
// split-K GEMV of lin_small_kernel with its A operand read from there;
// workgroup 0 also writes the residual, y and the MXFP4 rows to global
// memory for the step's later kernels.  The weight loads of a wave's first
// segment are issued before the norm, so they fly during it.
constexpr int kNormH = 2048;

struct NormLinArgs {
    const uint16_t* x;     // (M, H) bf16 residual stream
    const float* resid;    // (M, H) fp32 added as bf16 first (RESID)
    const uint16_t* nw;    // (H) bf16 norm weight
    float eps;
    uint16_t* x_out;       // workgroup 0: bf16(x + bf16(resid)) (RESID), may be null
    uint16_t* y;           // workgroup 0: the normed bf16 rows, may be null
    uint8_t* yq;           // workgroup 0: their MXFP4 rows (M, H/2) + (M, H/32), may be null
    uint8_t* ys;
    const uint8_t* wp;     // (N, H/2) + (N, H/32) weight
    const uint8_t* ws;
    float* out;            // (M, N) fp32
    int M, N, spw;
};

__device__ __forceinline__ void lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // LDS only: the weight loads stay in flight
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int R, int S, bool RESID>
__global__ __launch_bounds__(64 * R * S) void norm_lin_kernel(NormLinArgs a) {
    constexpr int H = kNormH, nch = H / 32, steps = nch / 4;
    __shared__ __align__(16) uint8_t lq[16][H / 2];
    __shared__ uint8_t lsc[16][nch];
    __shared__ float red[4][4];
    __shared__ mx::v4f redv[S > 1 ? S : 1][R][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int rt = wave % R, part = wave / R;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int n0 = (blockIdx.x * R + rt) * 16;
    const int M = a.M;
    const int sb = part * a.spw;
    const int se = min(steps, sb + a.spw);
    const bool act = n0 < a.N && sb < se;
    const int nrow = min(n0 + r, a.N - 1);
    const int arow = min(r, M - 1);
    const int boff = 4 * sb;
    const SegCtx cx{a.wp + (int64_t)nrow * (H / 2) + boff * 16, a.ws + (int64_t)nrow * nch + boff, nullptr, nullptr,
                    &lq[arow][boff * 16], &lsc[arow][boff], g, se - sb, nch - boff, true};
    SegBuf s0buf, s1buf;
    if (act) load_seg<A_SILU>(s0buf, cx, 0);
    // ---- the rows' norm, four rows a round (the norm weight is loaded with
    // the first rows, not after the reduction)
    const bool w0 = blockIdx.x == 0;
    uint4 wq4 = make_uint4(0, 0, 0, 0);
    if (tid < 256) wq4 = *reinterpret_cast<const uint4*>(a.nw + 8 * tid);
    for (int m0 = 0; m0 < M; m0 += 4) {
        float v[4][8];
        float ss[4] = {0.f, 0.f, 0.f, 0.f};
        if (tid < 256) {
            const int k0 = 8 * tid;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m0 + j;
                if (m >= M) continue;
                const int64_t rb = (int64_t)m * H;
                const uint4 q = *reinterpret_cast<const uint4*>(a.x + rb + k0);
                const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[j][2 * i] = mx::bf16_to_f32((uint16_t)(wq[i] & 0xFFFFu));
                    v[j][2 * i + 1] = mx::bf16_to_f32((uint16_t)(wq[i] >> 16));
                }
                if (RESID) {
                    const float4 o0 = *reinterpret_cast<const float4*>(a.resid + rb + k0);
                    const float4 o1 = *reinterpret_cast<const float4*>(a.resid + rb + k0 + 4);
                    const float of[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        v[j][i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(v[j][i] + mx::bf16_to_f32(mx::f32_to_bf16_rne(of[i]))));
                    if (w0 && a.x_out) {
                        uint32_t xo[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            xo[i] = (uint32_t)mx::f32_to_bf16_rne(v[j][2 * i]) |
                                    ((uint32_t)mx::f32_to_bf16_rne(v[j][2 * i + 1]) << 16);
                        *reinterpret_cast<uint4*>(a.x_out + rb + k0) = make_uint4(xo[0], xo[1], xo[2], xo[3]);
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) ss[j] = fmaf(v[j][i], v[j][i], ss[j]);
            }
            // the sum over the 256 threads in mxfp4_rmsnorm_quant's order
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ss[j] = mx::wave_sum_butterfly(ss[j]);
                if (lane == 0) red[j][wave] = ss[j];
            }
        }
        lds_sync();
        if (tid < 256) {
            const int k0 = 8 * tid;
            const uint32_t wq[4] = {wq4.x, wq4.y, wq4.z, wq4.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m0 + j;
                if (m >= M) continue;
                const float var = ((red[j][0] + red[j][1]) + (red[j][2] + red[j][3])) / (float)H;
                const float rr = 1.0f / sqrtf(var + a.eps);
                float yv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float wi = mx::bf16_to_f32((uint16_t)(wq[i / 2] >> (16 * (i & 1))));
                    const float t = mx::bf16_to_f32(mx::f32_to_bf16_rne(v[j][i] * rr));
                    yv[i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(t * wi));
                }
                float am = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(yv[i]));
                am = fmaxf(am, __shfl_xor(am, 1));
                am = fmaxf(am, __shfl_xor(am, 2));
                const uint32_t code = mx::e8m0_code(am);
                const uint32_t nib = mx::e2m1_pack8(yv, mx::e8m0_inv_scale(code));
                *reinterpret_cast<uint32_t*>(&lq[m][k0 / 2]) = nib;
                if ((tid & 3) == 0) lsc[m][k0 / 32] = (uint8_t)code;
                if (w0) {
                    const int64_t rb = (int64_t)m * H;
                    if (a.y) {
                        uint32_t yo[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            yo[i] = (uint32_t)mx::f32_to_bf16_rne(yv[2 * i]) | ((uint32_t)mx::f32_to_bf16_rne(yv[2 * i + 1]) << 16);
                        *reinterpret_cast<uint4*>(a.y + rb + k0) = make_uint4(yo[0], yo[1], yo[2], yo[3]);
                    }
                    if (a.yq) {
                        *reinterpret_cast<uint32_t*>(a.yq + (int64_t)m * (H / 2) + k0 / 2) = nib;
                        if ((tid & 3) == 0) a.ys[(int64_t)m * nch + k0 / 32] = (uint8_t)code;
                    }
                }
            }
        }
        lds_sync();   // red[] is reused by the next round; the LDS rows are complete
    }
    // ---- the GEMV (lin_small_kernel's), A from LDS
    mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (act) {
        for (int s0 = 0; s0 < cx.steps; s0 += 2 * kSeg) {
            if (s0 + kSeg < cx.steps) load_seg<A_SILU>(s1buf, cx, s0 + kSeg);
            acc = compute_seg<A_SILU>(s0buf, cx, s0, acc);
            if (s0 + kSeg >= cx.steps) break;
            if (s0 + 2 * kSeg < cx.steps) load_seg<A_SILU>(s0buf, cx, s0 + 2 * kSeg);
            acc = compute_seg<A_SILU>(s1buf, cx, s0 + kSeg, acc);
        }
    }
    if constexpr (S > 1) {
        redv[part][rt][lane] = acc;
        __syncthreads();
        if (part != 0) return;
#pragma unroll
        for (int p = 1; p < S; ++p) {
            const mx::v4f o = redv[p][rt][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += o[i];
        }
    }
    const int col = n0 + r;
    if (col >= a.N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * g + i;
        if (m < M) a.out[(int64_t)m * a.N + col] = acc[i];
    }
}

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ yd, int ystride,
                                                      const float* __restrict__ w, int E,
                                                      float* __restrict__ out, int M, int N) {
    const int m = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= N) return;
    const float* yb = yd + (int64_t)m * E * ystride;
    const float* wb = w + (int64_t)m * E;
    const int ee = E < 8 ? E : 8;  // src/ext/mxfp4_decode.cu:296 caps at 8 slots
    // every load issued before the first use (a use inside the loop made each
    // slot wait for the previous one's load), then the fmas in slot order
    float yv[8], wv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        yv[e] = e < ee ? yb[(int64_t)e * ystride + c] : 0.0f;
        wv[e] = e < ee ? wb[e] : 0.0f;
    }
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (e < ee) acc = fmaf(wv[e], yv[e], acc);
    out[(int64_t)m * N + c] = acc;
}

size_t silu_lds_bytes(int Kp) { return (size_t)16 * ((Kp >> 1) + (Kp >> 5)); }

template <class Tab>
int launch_gemv(const Tab& tab, const GemvArgs& a, int amode, hipStream_t st) {
    // one wave per workgroup when the 4-wave grid would not reach 4
    // workgroups per CU (the A_SILU tile build is shared by the waves of a
    // workgroup, so that path keeps 4)
    // (a 16-row tile with >= 4 MFMA K-steps is split over 4 waves by K, so a
    // tile's weight bytes are all in flight at once)
    const bool one = amode == A_FP4 && (int64_t)((a.N + 63) / 64) * a.T < 1024;
    const int steps = ((a.Kp >> 5) + 3) >> 2;
    if (one) {
        dim3 grid((unsigned)((a.N + 15) / 16), (unsigned)a.T);
        if (steps >= 4)
            hipLaunchKernelGGL((grouped_gemv_kernel<Tab, A_FP4, 1, 4>), grid, dim3(256), 0, st, tab, a);
        else
            hipLaunchKernelGGL((grouped_gemv_kernel<Tab, A_FP4, 1, 1>), grid, dim3(64), 0, st, tab, a);
    } else {
        dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)a.T);
        if (amode == A_FP4)
            hipLaunchKernelGGL((grouped_gemv_kernel<Tab, A_FP4, 4, 1>), grid, dim3(256), 0, st, tab, a);
        else if (steps >= 2) {
            // several column blocks per workgroup (h built once for them) when each
            // K part is one segment: fewer, fuller rounds of workgroups
            const int ncb = a.ncb > 1 && (steps + 1) / 2 <= kSeg ? a.ncb : 1;
            if (ncb > 1) {
                GemvArgs b = a;
                b.ncb = ncb;
                dim3 g2((unsigned)((a.N + 64 * ncb - 1) / (64 * ncb)), (unsigned)a.T);
                hipLaunchKernelGGL((grouped_gemv_kernel<Tab, A_SILU, 4, 2, true>), g2, dim3(512),
                                   silu_lds_bytes(a.Kp), st, tab, b);
            } else {
                hipLaunchKernelGGL((grouped_gemv_kernel<Tab, A_SILU, 4, 2>), grid, dim3(512), silu_lds_bytes(a.Kp),
                                   st, tab, a);
            }
        }
        else
            hipLaunchKernelGGL((grouped_gemv_kernel<Tab, A_SILU, 4, 1>), grid, dim3(256), silu_lds_bytes(a.Kp),
                               st, tab, a);
    }
    return mxh::launch_status("grouped_gemv");
}

// Runs a host table of T entries in launches of at most kMaxT entries.
int run_host_table(const uint8_t* const* wp_tab, const uint8_t* const* ws_tab, int T, GemvArgs a,
                   int amode, hipStream_t st) {
    for (int c0 = 0; c0 < T; c0 += kMaxT) {
        HostTable tab;
        const int n = (T - c0) < kMaxT ? (T - c0) : kMaxT;
        for (int i = 0; i < kMaxT; ++i) {
            tab.wp[i] = i < n ? wp_tab[c0 + i] : nullptr;
            tab.ws[i] = i < n ? ws_tab[c0 + i] : nullptr;
        }
        for (int i = 0; i < n; ++i)
            MXH_REQUIRE(tab.wp[i] && tab.ws[i], "pointer table entry %d is null", c0 + i);
        // grouping: entries with equal (weight, scale) pointers, in table order
        int nm = 0;
        for (int i = 0; i < kMaxT; ++i) {
            tab.info[i] = 0;
            tab.mem[i] = 0;
        }
        for (int i = 0; i < n; ++i) {
            bool seen = false;
            for (int j = 0; j < i && !seen; ++j) seen = tab.wp[j] == tab.wp[i] && tab.ws[j] == tab.ws[i];
            if (seen) continue;
            const int f = nm;
            for (int j = i; j < n; ++j)
                if (tab.wp[j] == tab.wp[i] && tab.ws[j] == tab.ws[i]) tab.mem[nm++] = (uint8_t)j;
            tab.info[i] = (uint32_t)(nm - f) | ((uint32_t)f << 8);
        }
        a.T = n;
        a.t0 = c0;
        // A_SILU: column blocks per workgroup so that the groups' workgroups
        // come to at most 512 (about one round, two per CU, and no fewer than 256)
        a.ncb = 1;
        if (amode == A_SILU) {
            int groups = 0;
            for (int i = 0; i < n; ++i) groups += tab.info[i] != 0;
            const int64_t total = (int64_t)groups * ((a.N + 63) / 64);
            while (a.ncb < 8 && total / a.ncb > 512) a.ncb *= 2;
        }
        const int rc = launch_gemv(tab, a, amode, st);
        if (rc != MXFP4_OK) return rc;
    }
    return MXFP4_OK;
}

int run_dev_table(const int64_t* wp_tab, const int64_t* ws_tab, int T, GemvArgs a, int amode,
                  hipStream_t st) {
    for (int c0 = 0; c0 < T; c0 += kMaxT) {
        DevTable tab{wp_tab + c0, ws_tab + c0};
        a.T = (T - c0) < kMaxT ? (T - c0) : kMaxT;
        a.t0 = c0;
        const int rc = launch_gemv(tab, a, amode, st);
        if (rc != MXFP4_OK) return rc;
    }
    return MXFP4_OK;
}

int check_common(int E, int M, int N, int K, int Kp, const char* op) {
    MXH_REQUIRE(E > 0 && M > 0 && N > 0 && K > 0, "%s: sizes must be positive (E=%d M=%d N=%d K=%d)", op, E, M, N, K);
    MXH_REQUIRE(Kp % 32 == 0 && Kp >= K, "%s: Kp=%d must be a multiple of 32 and >= K=%d", op, Kp, K);
    return MXFP4_OK;
}

}  // namespace

namespace mxh {
int lin_small(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc, float* y, int M, int N,
              int Kp, hipStream_t st);

// Small-M lin_pq: launches of up to 16 activation rows, each with R row
// tiles x S K-parts per workgroup, S the smallest power of two that gives
// the launch about 1024 waves (at most 16, and at most one part per MFMA
// K-step); R = 4 when K is not split.
int lin_pq_gemv(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc,
                float* y, int M, int N, int K, int Kp, hipStream_t st) {
    (void)K;
    for (int m0 = 0; m0 < M; m0 += 16) {
        const int rc = lin_small(xq + (int64_t)m0 * (Kp / 2), xsc + (int64_t)m0 * (Kp / 32), wp, wsc,
                                 y + (int64_t)m0 * N, M - m0 < 16 ? M - m0 : 16, N, Kp, st);
        if (rc != MXFP4_OK) return rc;
    }
    return MXFP4_OK;
}

int lin_small(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc, float* y, int M, int N,
              int Kp, hipStream_t st) {
    const int tiles = (N + 15) / 16;
    const int steps = (Kp / 32 + 3) / 4;
    int S = 1;
    while (S < 16 && 2 * S <= steps && (int64_t)tiles * S < 1024) S *= 2;
    const int spw = (steps + S - 1) / S;
    hipStream_t s = st;
#define MXH_LIN_SMALL(R_, S_)                                                                                 \
    hipLaunchKernelGGL((lin_small_kernel<R_, S_>), dim3((unsigned)((tiles + R_ - 1) / R_)), dim3(64 * R_ * S_), \
                       0, s, xq, xsc, wp, wsc, y, M, N, Kp, spw)
    switch (S) {
        case 1: MXH_LIN_SMALL(4, 1); break;
        case 2: MXH_LIN_SMALL(1, 2); break;
        case 4: MXH_LIN_SMALL(1, 4); break;
        case 8: MXH_LIN_SMALL(1, 8); break;
        default: MXH_LIN_SMALL(1, 16); break;
    }
#undef MXH_LIN_SMALL
    return launch_status("lin_pq_gemv");
}
}  // namespace mxh

extern "C" int mxfp4_moe_gateup(const uint8_t* xq, const uint8_t* xsc, const uint8_t* const* wp_tab,
                                const uint8_t* const* wsc_tab, float* gu, int E, int M, int N, int K,
                                int Kp, void* stream) {
    int rc = check_common(E, M, N, K, Kp, "moe_gateup");
    if (rc) return rc;
    MXH_REQUIRE(xq && xsc && wp_tab && wsc_tab && gu, "moe_gateup: null pointer");
    GemvArgs a{};
    a.E = E;
    a.map = MAP_GATEUP;
    a.N = N;
    a.K = K;
    a.Kp = Kp;
    a.aq = xq;
    a.as = xsc;
    a.out = gu;
    a.ld_out = 2 * (int64_t)N;
    return run_host_table(wp_tab, wsc_tab, 2 * E * M, a, A_FP4, mxh::as_stream(stream));
}

extern "C" int mxfp4_moe_gateup_devtab(const uint8_t* xq, const uint8_t* xsc, const int64_t* wp_tab,
                                       const int64_t* wsc_tab, float* gu, int E, int M, int N, int K,
                                       int Kp, void* stream) {
    int rc = check_common(E, M, N, K, Kp, "moe_gateup_tab");
    if (rc) return rc;
    MXH_REQUIRE(xq && xsc && wp_tab && wsc_tab && gu, "moe_gateup_tab: null pointer");
    GemvArgs a{};
    a.E = E;
    a.map = MAP_GATEUP;
    a.N = N;
    a.K = K;
    a.Kp = Kp;
    a.aq = xq;
    a.as = xsc;
    a.out = gu;
    a.ld_out = 2 * (int64_t)N;
    return run_dev_table(wp_tab, wsc_tab, 2 * E * M, a, A_FP4, mxh::as_stream(stream));
}

extern "C" int mxfp4_moe_down(const float* gu, const uint8_t* const* wp_tab, const uint8_t* const* wsc_tab,
                              float* yd, int E, int M, int N, int K, int Kp, void* stream) {
    int rc = check_common(E, M, N, K, Kp, "moe_down");
    if (rc) return rc;
    MXH_REQUIRE(gu && wp_tab && wsc_tab && yd, "moe_down: null pointer");
    MXH_REQUIRE(Kp <= 4096, "moe_down: Kp=%d exceeds the 4096 supported by the LDS tile", Kp);
    GemvArgs a{};
    a.E = E;
    a.map = MAP_PLAIN;
    a.N = N;
    a.K = K;
    a.Kp = Kp;
    a.gu = gu;
    a.out = yd;
    a.ld_out = N;
    return run_host_table(wp_tab, wsc_tab, E * M, a, A_SILU, mxh::as_stream(stream));
}

extern "C" int mxfp4_moe_down_devtab(const float* gu, const int64_t* wp_tab, const int64_t* wsc_tab,
                                     float* yd, int E, int M, int N, int K, int Kp, void* stream) {
    int rc = check_common(E, M, N, K, Kp, "moe_down_tab");
    if (rc) return rc;
    MXH_REQUIRE(gu && wp_tab && wsc_tab && yd, "moe_down_tab: null pointer");
    MXH_REQUIRE(Kp <= 4096, "moe_down_tab: Kp=%d exceeds the 4096 supported by the LDS tile", Kp);
    GemvArgs a{};
    a.E = E;
    a.map = MAP_PLAIN;
    a.N = N;
    a.K = K;
    a.Kp = Kp;
    a.gu = gu;
    a.out = yd;
    a.ld_out = N;
    return run_dev_table(wp_tab, wsc_tab, E * M, a, A_SILU, mxh::as_stream(stream));
}

extern "C" int mxfp4_moe_combine(const float* yd, int ystride, const float* w, int E, float* out, int M,
                                 int N, void* stream) {
    MXH_REQUIRE(yd && w && out, "moe_combine: null pointer");
    MXH_REQUIRE(M > 0 && E > 0 && N > 0, "moe_combine: sizes must be positive (M=%d E=%d N=%d)", M, E, N);
    MXH_REQUIRE(ystride >= N, "moe_combine: ystride %d < N %d", ystride, N);
    dim3 grid((unsigned)((N + 255) / 256), (unsigned)M);
    hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, mxh::as_stream(stream), yd, ystride, w, E, out, M, N);
    return mxh::launch_status("moe_combine");
}

extern "C" int mxfp4_rmsnorm_lin_pq(const void* x, const float* resid, const void* norm_w, float eps, int M, int H,
                                    void* x_out, void* y, uint8_t* yq, uint8_t* ys, const uint8_t* wp,
                                    const uint8_t* wsc, int N, float* out, void* stream) {
    MXH_REQUIRE(x && norm_w && wp && wsc && out, "rmsnorm_lin_pq: null pointer");
    MXH_REQUIRE(H == kNormH, "rmsnorm_lin_pq: H=%d (this kernel is built for %d)", H, kNormH);
    MXH_REQUIRE(M >= 1 && M <= 16 && N > 0, "rmsnorm_lin_pq: M=%d (1..16) N=%d", M, N);
    MXH_REQUIRE(!yq == !ys, "rmsnorm_lin_pq: yq and ys go together");
    MXH_REQUIRE(resid || !x_out, "rmsnorm_lin_pq: x_out needs resid");
    MXH_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && (!resid || ((uintptr_t)resid & 15) == 0) &&
                    (!x_out || ((uintptr_t)x_out & 15) == 0) && (!y || ((uintptr_t)y & 15) == 0) &&
                    (!yq || ((uintptr_t)yq & 3) == 0) && ((uintptr_t)wp & 15) == 0,
                "rmsnorm_lin_pq: x, resid, norm_w, x_out, y, wp must be 16-byte aligned, yq 4-byte");
    const int tiles = (N + 15) / 16;
    const int steps = kNormH / 128;
    int S = 1;
    while (S < 16 && 2 * S <= steps && (int64_t)tiles * S < 1024) S *= 2;
    NormLinArgs a{static_cast<const uint16_t*>(x), resid, static_cast<const uint16_t*>(norm_w), eps,
                  static_cast<uint16_t*>(x_out), static_cast<uint16_t*>(y), yq, ys, wp, wsc, out, M, N,
                  (steps + S - 1) / S};
    hipStream_t st = mxh::as_stream(stream);
#define MXH_NORM_LIN(R_, S_)                                                                                       \
    do {                                                                                                           \
        if (resid)                                                                                                 \
            hipLaunchKernelGGL((norm_lin_kernel<R_, S_, true>), dim3((unsigned)((tiles + R_ - 1) / R_)),          \
                               dim3(64 * R_ * S_), 0, st, a);                                                      \
        else                                                                                                       \
            hipLaunchKernelGGL((norm_lin_kernel<R_, S_, false>), dim3((unsigned)((tiles + R_ - 1) / R_)),         \
                               dim3(64 * R_ * S_), 0, st, a);                                                      \
    } while (0)
    switch (S) {
        case 1: MXH_NORM_LIN(4, 1); break;
        case 2: MXH_NORM_LIN(1, 2); break;
        case 4: MXH_NORM_LIN(1, 4); break;
        case 8: MXH_NORM_LIN(1, 8); break;
        default: MXH_NORM_LIN(1, 16); break;
    }
#undef MXH_NORM_LIN
    return mxh::launch_status("rmsnorm_lin_pq");
}
