// gemm2.hip -- block-scaled MXFP4 x MXFP4 GEMM for large prefill shapes.
//
// y (M, N) fp32 = A (M, Kp) * W (N, Kp)^T, both operands packed E2M1 rows with
// E8M0 32-block scales (the lin_pq contract, src/ext/mxfp4_decode.cu:135-170).
// Used when Kp is a multiple of 256 and M > 16.
//
// * Workgroup tile BM x BN with NW waves in 2 (M) x NW/2 (N).  For large
//   grids 256 x 256 with 8 waves: a wave owns 128 x 64 as 4 x 2
//   v_mfma_scale_f32_32x32x64_f8f6f4 accumulators.  (NW = 4, 128 x 128 per
//   wave with the accumulators in AGPRs, would read a third less from LDS but
//   does not fit the register file without spills.)  Smaller grids take
//   128 x 128 or 64 x 64 tiles with 4 waves and a deeper ring (the launcher
//   picks the instance); every instance runs the same MFMA chain per output.
// * K step BK (BK/2 bytes of each operand row; BK = 256 here).  Global -> LDS
//   with buffer_load_dwordx4 ... lds (no registers, no repacking): lane i of an
//   instruction writes LDS bytes [16i, 16i+16) of a 1 KB block of whole rows.
//   The lane loads the global 16-byte chunk that belongs at its LDS slot under
//   an XOR swizzle, chosen so that the 16 lanes of one ds_read_b128 phase
//   (16 consecutive rows, one chunk each, 256 bytes over the 64 banks) hit 16
//   different 16-byte bank groups.
// * NSTAGE stages in a ring, one workgroup per CU: the copies of the next
//   NSTAGE-1 steps are in flight during the MFMAs of a step.  A step's copies
//   are spread over its four MFMA substeps (issued in one burst they held
//   back each wave's MFMAs while the memory pipeline accepted them).  Every
//   wave issues the same number of copies per step, so a step's arrival is a
//   fixed vmcnt.
// * Measured limit (MI355X, 4096 x 4096 x 2048, timing copies that drop one
//   part): a 256-wide K step takes ~2.0 us, and each of its three parts
//   alone takes 1.5-1.6 us -- the L2 -> LDS copies (68 KB per CU, ~42 GB/s
//   per CU when all 256 CUs copy), the LDS operand reads with the MFMAs, and
//   the MFMAs alone at the power-limited ~1.8 GHz clock (1.14 us) -- so the
//   step is bound by all three at once, not by LDS bank conflicts (none).
// * Scales: BK/32 bytes per row per step, loaded the same way (4 bytes per
//   lane) and permuted once per step (v_perm_b32) so that op_sel = ks selects
//   the byte of K-substep ks.
// * XCD-aware order: workgroup b runs on XCD b % 8; each XCD gets a compact
//   block of tiles (a few tile rows by a few tile columns), so the A and W
//   K-slabs of one step are fetched into that XCD's L2 once and shared.
#include "lds_dma.h"
#include "mx_device.h"
#include "mx_host.h"

namespace {

template <int BM, int BN, int BK, int NW>
struct Tile {
    static constexpr int WM = BM / 2;                     // rows per wave (2 waves along M)
    static constexpr int IM = WM / 32;                    // 32-row accumulator tiles per wave
    static constexpr int ROWB = BK / 2;                   // data bytes per row per step
    static constexpr int CPR = ROWB / 16;                 // 16-byte chunks per row
    static constexpr int RPB = 1024 / ROWB;               // rows per 1 KB copy block
    static constexpr int SCB = BK / 32;                   // scale bytes per row per step
    static constexpr int KS = BK / 64;                    // MFMA K-substeps per step
    static constexpr int A_BYTES = BM * ROWB;
    static constexpr int W_BYTES = BN * ROWB;
    static constexpr int S_BYTES = (BM + BN) * SCB;
    static constexpr int STAGE = A_BYTES + W_BYTES + S_BYTES;
    static constexpr int NTHREADS = 64 * NW;
    static constexpr int WN_W = NW / 2;                   // waves along N (2 along M)
    static constexpr int WCOLS = BN / WN_W;               // columns per wave
    static constexpr int TN = WCOLS / 32;                 // 32-col accumulator tiles per wave
    static constexpr int A_CP = A_BYTES / 1024 / NW;      // A copies per wave per step
    static constexpr int W_CP = W_BYTES / 1024 / NW;
    static constexpr int S_Q = S_BYTES / 256;             // scale copies (4 bytes x 64 lanes)
    static constexpr int S_CP = (S_Q + NW - 1) / NW;
    static constexpr int COPIES = A_CP + W_CP + S_CP;
    static_assert(CPR == 4 || CPR == 8, "BK 128 or 256");
    static_assert(A_BYTES % (1024 * NW) == 0 && W_BYTES % (1024 * NW) == 0 && S_BYTES % 256 == 0, "copy split");
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
};

struct G2Args {
    const uint8_t* aq;
    const uint8_t* as;
    const uint8_t* wp;
    const uint8_t* ws;
    float* y;
    int M, N, Kp;
    int tiles_m, tiles_n;
    int bm, bn;         // XCD block: bm tile rows x bn tile columns
    int xblk_n;         // XCD blocks along N
    int per_xcd;        // workgroups per XCD (grid = 8 * per_xcd)
};

using mx::buf_rsrc;
using mx::dma16;
using mx::dma4;
using mx::lds_addr;
using mx::v4u;

// Swizzle of row r: the LDS slot of logical chunk c is c ^ swz_key(r).  A
// ds_read_b128 phase covers 16 consecutive rows (16-aligned) at one logical
// chunk, 256 bytes over all 64 banks; the rows of the phase that sit at the
// same position of a 256-byte bank line (same r mod 256/ROWB) get distinct
// keys.  The key depends on r mod 16 only (the operand reads rely on it).
// The copies write whole 1 KB blocks, so they never conflict.
template <int CPR>
__device__ __forceinline__ int swz_key(int r) {
    if constexpr (CPR == 8) return mx::swz_key128(r);
    else return ((r >> 1) ^ (r >> 2)) & 3;
}

// Per-tile copy state: descriptors of the tile's A / W rows and scale rows,
// and the lane's byte offsets within them.
struct CopyState {
    v4u ra, rw, rsa, rsw;
    uint32_t va[2], vw[2];   // lane offset of A / W copies with an even / odd index
    uint32_t vs;             // lane offset of scale copies
};

template <int BM, int BN, int BK, int NW>
__device__ __forceinline__ CopyState copy_state(const G2Args& g, int m0, int n0) {
    using T = Tile<BM, BN, BK, NW>;
    const int w = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int64_t cbytes = g.Kp >> 1, nch = g.Kp >> 5;
    CopyState c;
    c.ra = buf_rsrc(g.aq + m0 * cbytes, (int64_t)(g.M - m0) * cbytes);
    c.rw = buf_rsrc(g.wp + n0 * cbytes, (int64_t)(g.N - n0) * cbytes);
    c.rsa = buf_rsrc(g.as + m0 * nch, (int64_t)(g.M - m0) * nch);
    c.rsw = buf_rsrc(g.ws + n0 * nch, (int64_t)(g.N - n0) * nch);
    const int lrow = l / T::CPR, slot = l % T::CPR;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        // copy j of the wave covers rows (w*CP + j)*RPB + lrow; with an even
        // CP the swizzle key (row mod 16) depends on j only through its parity
        const int ra = (w * T::A_CP + p) * T::RPB + lrow;
        const int rw = (w * T::W_CP + p) * T::RPB + lrow;
        c.va[p] = (uint32_t)(ra * cbytes + ((slot ^ swz_key<T::CPR>(ra)) << 4)) - (uint32_t)(p * T::RPB * cbytes);
        c.vw[p] = (uint32_t)(rw * cbytes + ((slot ^ swz_key<T::CPR>(rw)) << 4)) - (uint32_t)(p * T::RPB * cbytes);
    }
    constexpr int LPR = T::SCB / 4;   // lanes per scale row
    c.vs = (uint32_t)((l / LPR) * nch + 4 * (l % LPR));
    return c;
}

// The global -> LDS copies of K-step k0 (elements) into stage `buf`, in KS
// parts: part q issues the copies c with c % KS == q of the wave's
// Tile::COPIES (A blocks, then W blocks, then scales), so that the copies of
// the next step are spread over the MFMA substeps of this one (a wave issues
// in order, so copies issued in one burst hold back its MFMAs while the
// memory pipeline accepts them).
template <int BM, int BN, int BK, int NW>
__device__ __forceinline__ void issue_part(const G2Args& g, const CopyState& c, uint32_t buf, int k0, int part) {
    using T = Tile<BM, BN, BK, NW>;
    static_assert(T::A_CP % 2 == 0 && T::W_CP % 2 == 0, "even copy counts (swizzle key parity)");
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar selects below
    const uint32_t cbytes = g.Kp >> 1, nch = g.Kp >> 5;
#pragma unroll
    for (int j = 0; j < T::A_CP; ++j) {
        if (j % T::KS != part) continue;
        const int blk = w * T::A_CP + j;   // c.va holds the wave's first block; soffset adds block j
        dma16(c.va[j & 1], c.ra, (uint32_t)(j * T::RPB) * cbytes + (k0 >> 1), buf + blk * 1024);
    }
#pragma unroll
    for (int j = 0; j < T::W_CP; ++j) {
        if ((T::A_CP + j) % T::KS != part) continue;
        const int blk = w * T::W_CP + j;
        dma16(c.vw[j & 1], c.rw, (uint32_t)(j * T::RPB) * cbytes + (k0 >> 1), buf + T::A_BYTES + blk * 1024);
    }
    // scales: rows 0..BM-1 of A then 0..BN-1 of W, SCB bytes each, 4 bytes a
    // lane; waves past the last copy rewrite an earlier one (same bytes)
    constexpr int LPR = T::SCB / 4;
#pragma unroll
    for (int j = 0; j < T::S_CP; ++j) {
        if ((T::A_CP + T::W_CP + j) % T::KS != part) continue;
        const int q = (w * T::S_CP + j) % T::S_Q;
        const int row0 = q * 64 / LPR;          // first row of the copy
        const bool is_a = row0 < BM;
        v4u rs;
        rs.x = __builtin_amdgcn_readfirstlane(is_a ? c.rsa.x : c.rsw.x);
        rs.y = __builtin_amdgcn_readfirstlane(is_a ? c.rsa.y : c.rsw.y);
        rs.z = __builtin_amdgcn_readfirstlane(is_a ? c.rsa.z : c.rsw.z);
        rs.w = 0x00020000u;
        dma4(c.vs, rs, (uint32_t)((is_a ? row0 : row0 - BM)) * nch + (k0 >> 5),
             buf + T::A_BYTES + T::W_BYTES + q * 256);
    }
}

template <int BM, int BN, int BK, int NW>
__device__ __forceinline__ void issue_stage(const G2Args& g, const CopyState& c, uint32_t buf, int k0) {
#pragma unroll
    for (int q = 0; q < Tile<BM, BN, BK, NW>::KS; ++q) issue_part<BM, BN, BK, NW>(g, c, buf, k0, q);
}

template <int OP>
__device__ __forceinline__ mx::v16f mfma32(uint4 a, uint4 b, mx::v16f c, uint32_t sa, uint32_t sb) {
    mx::v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    mx::v8i bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 4, 4, OP, (int)sa, OP, (int)sb);
}

// Scale word of this lane: byte ks = block 2*ks + h of the step.
template <int SCB>
__device__ __forceinline__ uint32_t scale_word(const uint8_t* srow, int h) {
    if constexpr (SCB == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(srow);
        return __builtin_amdgcn_perm(v.y, v.x, h ? 0x07050301u : 0x06040200u);
    } else {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(srow);
        return __builtin_amdgcn_perm(v, v, h ? 0x0C0C0301u : 0x0C0C0200u);
    }
}

// The MFMAs of one step on the stage at `cur`.  The rows a lane reads,
// wm*128 + i*32 + lr and wn*BN/4 + j*32 + lr, differ from lr by multiples of
// 16, so their swizzle key is swz_key(lr): one LDS address per operand and
// K-substep, the row offsets are immediates.
template <int BM, int BN, int BK, int NW>
__device__ __forceinline__ void mfma_step(const uint8_t* cur, mx::v16f (&acc)[Tile<BM, BN, BK, NW>::IM][Tile<BM, BN, BK, NW>::TN], const G2Args& g,
                                          const CopyState& cs, uint32_t nxt, int k_next) {
    using T = Tile<BM, BN, BK, NW>;
    constexpr int TN = T::TN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave / T::WN_W, wn = wave % T::WN_W;
    const int lr = lane & 31;
    const int h = lane >> 5;
    const int key = swz_key<T::CPR>(lr);
    const uint8_t* la = cur + (wm * T::WM + lr) * T::ROWB;
    const uint8_t* lw = cur + T::A_BYTES + (wn * T::WCOLS + lr) * T::ROWB;
    const uint8_t* lsa = cur + T::A_BYTES + T::W_BYTES + (wm * T::WM + lr) * T::SCB;
    const uint8_t* lsw = cur + T::A_BYTES + T::W_BYTES + BM * T::SCB + (wn * T::WCOLS + lr) * T::SCB;
    uint32_t sa[T::IM], sb[TN];
#pragma unroll
    for (int i = 0; i < T::IM; ++i) sa[i] = scale_word<T::SCB>(lsa + i * 32 * T::SCB, h);
#pragma unroll
    for (int j = 0; j < TN; ++j) sb[j] = scale_word<T::SCB>(lsw + j * 32 * T::SCB, h);
    // operand registers of two substeps: the reads of substep ks+1 are issued
    // before the MFMAs of substep ks, so their LDS latency hides under them
    uint4 af[2][T::IM], bf[2][TN];
    auto load = [&](int ks, int r) {
        const int koff = ((2 * ks + h) ^ key) << 4;
#pragma unroll
        for (int i = 0; i < T::IM; ++i) af[r][i] = *reinterpret_cast<const uint4*>(la + koff + i * 32 * T::ROWB);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[r][j] = *reinterpret_cast<const uint4*>(lw + koff + j * 32 * T::ROWB);
    };
    load(0, 0);
#pragma unroll
    for (int ks = 0; ks < T::KS; ++ks) {
        // keep each substep's copies, operand reads and MFMAs together (the
        // scheduler would otherwise hoist every copy ahead of the MFMAs)
        __builtin_amdgcn_sched_barrier(0);
        issue_part<BM, BN, BK, NW>(g, cs, nxt, k_next, ks);
        if (ks + 1 < T::KS) load(ks + 1, (ks + 1) & 1);
        const int r = ks & 1;
#pragma unroll
        for (int i = 0; i < T::IM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if (ks == 0) acc[i][j] = mfma32<0>(af[r][i], bf[r][j], acc[i][j], sa[i], sb[j]);
                if (ks == 1) acc[i][j] = mfma32<1>(af[r][i], bf[r][j], acc[i][j], sa[i], sb[j]);
                if (ks == 2) acc[i][j] = mfma32<2>(af[r][i], bf[r][j], acc[i][j], sa[i], sb[j]);
                if (ks == 3) acc[i][j] = mfma32<3>(af[r][i], bf[r][j], acc[i][j], sa[i], sb[j]);
            }
    }
}

template <int BM, int BN, int BK, int NSTAGE, int NW>
__global__ __launch_bounds__(64 * NW, 1) void gemm2_kernel(G2Args g) {
    using T = Tile<BM, BN, BK, NW>;
    constexpr int TN = T::TN;
    static_assert(NSTAGE >= 2 && NSTAGE * T::STAGE <= 160 * 1024, "LDS ring");
    __shared__ __align__(16) uint8_t ring[NSTAGE * T::STAGE];

    // XCD-major tile order: XCD x = bid % 8 takes the blocks x, x+8, ... of
    // bm x bn tiles; within a block, tiles go along N first
    const int bid = blockIdx.x;
    const int xcd = bid & 7;
    const int k = bid >> 3;                                 // index within the XCD
    const int per_blk = g.bm * g.bn;
    const int xb = xcd + 8 * (k / per_blk);                 // XCD block number
    const int in = k % per_blk;
    const int tm = (xb / g.xblk_n) * g.bm + in / g.bn;
    const int tn = (xb % g.xblk_n) * g.bn + in % g.bn;
    if (tm >= g.tiles_m || tn >= g.tiles_n) return;
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave / T::WN_W, wn = wave % T::WN_W;
    const int lr = lane & 31;
    const int h = lane >> 5;
    const int nsteps = g.Kp / BK;

    mx::v16f acc[T::IM][TN];
#pragma unroll
    for (int i = 0; i < T::IM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const CopyState cs = copy_state<BM, BN, BK, NW>(g, m0, n0);
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(ring));   // LDS byte address of the ring
#pragma unroll
    for (int s = 0; s < NSTAGE - 1; ++s) issue_stage<BM, BN, BK, NW>(g, cs, ring_lds + s * T::STAGE, min(s, nsteps - 1) * BK);

    for (int it0 = 0; it0 < nsteps; it0 += NSTAGE) {
#pragma unroll
        for (int s = 0; s < NSTAGE; ++s) {
            const int it = it0 + s;
            if (it < nsteps) {
                // this wave's copies of step it have landed (those of the
                // NSTAGE-2 later steps may still be in flight) and its LDS
                // reads of step it-1 are done; after the barrier every wave's.
                // Every step issues one stage of copies (past the last step
                // they re-read the last K slab into a free stage), so the
                // count is the same at every step.
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 2) * T::COPIES) : "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                // MFMAs on this step's stage; the stage step it-1 used is
                // refilled with step it+NSTAGE-1, spread over the substeps
                mfma_step<BM, BN, BK, NW>(ring + s * T::STAGE, acc, g, cs, ring_lds + ((s + NSTAGE - 1) % NSTAGE) * T::STAGE,
                                  min(it + NSTAGE - 1, nsteps - 1) * BK);
            }
        }
    }

    // the copies issued past the last step must land before the workgroup's
    // LDS can be handed to another workgroup
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < T::IM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if constexpr (NW == 4) mx::pin_acc(acc[i][j]);
            else mx::pin(acc[i][j]);
        }
    // accumulator element e of lane l: row 8*(e/4) + 4*(l/32) + e%4, column l%32;
    // non-temporal stores (y is not read back by this launch; measured:
    // 2048 x 2048 x 768 9.2 -> 7.9 us)
#pragma unroll
    for (int i = 0; i < T::IM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * T::WCOLS + j * 32 + lr;
            if (col >= g.N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * T::WM + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (row < g.M) __builtin_nontemporal_store(acc[i][j][e], g.y + (int64_t)row * g.N + col);
            }
        }
}

// Picks the XCD block (bm x bn tiles) for a tile grid: about an eighth of the
// tiles per XCD, as square as the grid allows.
void xcd_blocks(G2Args& g) {
    const int nt = g.tiles_m * g.tiles_n;
    const int want = (nt + 7) / 8;
    int bm = 1;
    while (bm * 2 <= g.tiles_m && (bm * 2) * (bm * 2) <= want) bm *= 2;
    int bn = (want + bm - 1) / bm;
    if (bn > g.tiles_n) bn = g.tiles_n;
    g.bm = bm;
    g.bn = bn;
    g.xblk_n = (g.tiles_n + bn - 1) / bn;
    const int xblk_m = (g.tiles_m + bm - 1) / bm;
    const int nblk = xblk_m * g.xblk_n;
    g.per_xcd = ((nblk + 7) / 8) * bm * bn;
}

}  // namespace

namespace mxh {
// Any M > 16 with Kp a multiple of 256 (the buffer descriptors address each
// operand with 32-bit byte offsets, hence the size bound).
bool lin_pq_gemm2_supported(int M, int N, int Kp) {
    const bool fits = (int64_t)M * (Kp / 2) < (1ll << 32) && (int64_t)N * (Kp / 2) < (1ll << 32);
    return M > 16 && N > 0 && Kp >= 256 && (Kp % 256) == 0 && fits;
}

template <int BM, int BN, int BK, int NSTAGE, int NW>
int launch_gemm2(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc, float* y, int M, int N,
                 int Kp, hipStream_t st) {
    MXH_REQUIRE(Kp % BK == 0, "lin_pq_gemm2: Kp=%d is not a multiple of %d", Kp, BK);
    G2Args g{xq, xsc, wp, wsc, y, M, N, Kp, 0, 0, 0, 0, 0, 0};
    g.tiles_m = (M + BM - 1) / BM;
    g.tiles_n = (N + BN - 1) / BN;
    xcd_blocks(g);
    hipLaunchKernelGGL((gemm2_kernel<BM, BN, BK, NSTAGE, NW>), dim3(8 * g.per_xcd), dim3(64 * NW), 0, st, g);
    return launch_status("lin_pq_gemm2");
}

int lin_pq_gemm2(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc, float* y,
                 int M, int N, int Kp, hipStream_t st) {
    MXH_REQUIRE(((uintptr_t)xq & 15) == 0 && ((uintptr_t)wp & 15) == 0,
                "lin_pq: packed operands must be 16-byte aligned");
    MXH_REQUIRE(((uintptr_t)xsc & 3) == 0 && ((uintptr_t)wsc & 3) == 0,
                "lin_pq: scale rows must be 4-byte aligned");
    // Tile by grid size: 256 x 256 (2 stages) when it gives at least 128
    // tiles; else 128 x 128 (4 stages) when that gives at least 192; else
    // 64 x 64 with 8 stages, i.e. up to 7 K-steps of copies in flight, so a
    // small grid pays about one memory latency instead of one per K-step --
    // or with 4 stages (two workgroups per CU) when one per CU would take
    // two rounds.  Measured on MI355X: 512 x 1536 x 2048 in 6.5 us against
    // 11.1 us for the 128 x 128 register-staged GEMM; all tiles give the same
    // bits (the same MFMA chain per output).
    const int64_t t256 = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
    const int64_t t64 = (int64_t)((M + 63) / 64) * ((N + 63) / 64);
    if (t256 >= 128) return launch_gemm2<256, 256, 256, 2, 8>(xq, xsc, wp, wsc, y, M, N, Kp, st);
    if (t128 >= 192) return launch_gemm2<128, 128, 256, 4, 4>(xq, xsc, wp, wsc, y, M, N, Kp, st);
    if (t64 > 256) return launch_gemm2<64, 64, 256, 4, 4>(xq, xsc, wp, wsc, y, M, N, Kp, st);
    return launch_gemm2<64, 64, 256, 8, 4>(xq, xsc, wp, wsc, y, M, N, Kp, st);
}
}  // namespace mxh
