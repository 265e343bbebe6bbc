// gemm2.hip -- block-scaled MXFP4 x MXFP4 GEMM for large prefill shapes.
//
// y (M, N) fp32 = A (M, Kp) * W (N, Kp)^T, both operands packed E2M1 rows with
// E8M0 32-block scales (the lin_pq contract, src/ext/mxfp4_decode.cu:135-170).
// Used when Kp is a multiple of 256, M > 16 and the grid has at least 128 tiles.
//
// * Workgroup tile 256 x BN (BN = 256 here), 8 waves in 2 (M) x 4 (N); a
//   wave owns 128 x BN/4 as 4 x BN/128 v_mfma_scale_f32_32x32x64_f8f6f4
//   accumulators.
// * K step BK (BK/2 bytes of each operand row; BK = 256 here).  Global -> LDS with
//   global_load_lds_dwordx4 (no registers, no repacking): lane i of an
//   instruction writes LDS bytes [16i, 16i+16) of a 1 KB block of whole rows.
//   The lane loads the global 16-byte chunk that belongs at its LDS slot under
//   an XOR swizzle, chosen so that the 16 lanes of one ds_read_b128 phase
//   (16 consecutive rows, one chunk each, 256 bytes over the 64 banks) hit 16
//   different 16-byte bank groups.
// * NSTAGE stages in a ring, one workgroup per CU: the copies of the next
//   NSTAGE-1 steps are in flight during the MFMAs of a step.  Every wave
//   issues the same number of copies per step, so a step's arrival is a fixed
//   vmcnt.
// * Scales: BK/32 bytes per row per step, loaded the same way (4 bytes per
//   lane) and permuted once per step (v_perm_b32) so that op_sel = ks selects
//   the byte of K-substep ks.
// * XCD-aware order: workgroup b runs on XCD b % 8; each XCD gets a compact
//   block of tiles (a few tile rows by a few tile columns), so the A and W
//   K-slabs of one step are fetched into that XCD's L2 once and shared.
#include "mx_device.h"
#include "mx_host.h"

namespace {

constexpr int BM = 256;
constexpr int NTHREADS = 512;

template <int BN, int BK>
struct Tile {
    static constexpr int ROWB = BK / 2;                   // data bytes per row per step
    static constexpr int CPR = ROWB / 16;                 // 16-byte chunks per row
    static constexpr int RPB = 1024 / ROWB;               // rows per 1 KB copy block
    static constexpr int SCB = BK / 32;                   // scale bytes per row per step
    static constexpr int KS = BK / 64;                    // MFMA K-substeps per step
    static constexpr int A_BYTES = BM * ROWB;
    static constexpr int W_BYTES = BN * ROWB;
    static constexpr int S_BYTES = (BM + BN) * SCB;
    static constexpr int STAGE = A_BYTES + W_BYTES + S_BYTES;
    static constexpr int TN = BN / 128;                   // 32-col accumulator tiles per wave
    static constexpr int A_CP = A_BYTES / 1024 / 8;       // A copies per wave per step
    static constexpr int W_CP = W_BYTES / 1024 / 8;
    static constexpr int S_Q = S_BYTES / 256;             // scale copies (4 bytes x 64 lanes)
    static constexpr int S_CP = (S_Q + 7) / 8;
    static constexpr int COPIES = A_CP + W_CP + S_CP;
    static_assert(CPR == 4 || CPR == 8, "BK 128 or 256");
    static_assert(A_BYTES % 8192 == 0 && W_BYTES % 8192 == 0 && S_BYTES % 256 == 0, "copy split");
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

// Global -> LDS copies, written as inline asm on purpose: the compiler's
// own wait insertion treats any pending LDS copy as aliasing every later LDS
// read and would wait for all of them (vmcnt(0)) before the first operand read
// of a step, collapsing the stage ring.  The copies are waited for explicitly
// (s_waitcnt vmcnt(n) before each step's barrier).  The LDS address goes in M0,
// which is saved and restored around the copy.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}
__device__ __forceinline__ void dma16(const void* src, uint8_t* dst) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr(dst)))
                 : "memory");
}
__device__ __forceinline__ void dma4(const void* src, uint8_t* dst) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_addr(dst)))
                 : "memory");
}

// Swizzle of row r: the LDS slot of logical chunk c is c ^ swz_key(r).  A
// ds_read_b128 phase covers 16 consecutive rows (16-aligned) at one logical
// chunk, 256 bytes over all 64 banks; the rows of the phase that sit at the
// same position of a 256-byte bank line (same r mod 256/ROWB) get distinct
// keys.  The key depends on r mod 16 only (the operand reads rely on it).
// The copies write whole 1 KB blocks, so they never conflict.
template <int CPR>
__device__ __forceinline__ int swz_key(int r) {
    if constexpr (CPR == 8) return (r & 7) ^ ((r >> 3) & 1);
    else return ((r >> 1) ^ (r >> 2)) & 3;
}

// Issues the global -> LDS copies of K-step k0 (elements) into stage `buf`:
// Tile::COPIES instructions per wave.
template <int BN, int BK>
__device__ __forceinline__ void issue_stage(const G2Args& g, uint8_t* buf, int m0, int n0, int k0) {
    using T = Tile<BN, BK>;
    const int w = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int cbytes = g.Kp >> 1;
    const int nch = g.Kp >> 5;
    const int lrow = l / T::CPR;
    const int slot = l % T::CPR;
#pragma unroll
    for (int j = 0; j < T::A_CP; ++j) {
        const int blk = w * T::A_CP + j;
        const int row = blk * T::RPB + lrow;
        const int c = slot ^ swz_key<T::CPR>(row);
        dma16(g.aq + (int64_t)min(m0 + row, g.M - 1) * cbytes + (k0 >> 1) + c * 16, buf + blk * 1024);
    }
#pragma unroll
    for (int j = 0; j < T::W_CP; ++j) {
        const int blk = w * T::W_CP + j;
        const int row = blk * T::RPB + lrow;
        const int c = slot ^ swz_key<T::CPR>(row);
        dma16(g.wp + (int64_t)min(n0 + row, g.N - 1) * cbytes + (k0 >> 1) + c * 16,
              buf + T::A_BYTES + blk * 1024);
    }
    // scales: rows 0..BM-1 of A then 0..BN-1 of W, SCB bytes each, 4 bytes a
    // lane; waves past the last copy rewrite an earlier one (same bytes)
    constexpr int LPR = T::SCB / 4;                       // lanes per row
#pragma unroll
    for (int j = 0; j < T::S_CP; ++j) {
        const int q = (w * T::S_CP + j) % T::S_Q;
        const int wi = q * 64 + l;
        const int row = wi / LPR;
        const int part = wi % LPR;
        const uint8_t* src = row < BM ? g.as + (int64_t)min(m0 + row, g.M - 1) * nch
                                      : g.ws + (int64_t)min(n0 + row - BM, g.N - 1) * nch;
        dma4(src + (k0 >> 5) + 4 * part, buf + T::A_BYTES + T::W_BYTES + q * 256);
    }
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
template <int BN, int BK>
__device__ __forceinline__ void mfma_step(const uint8_t* cur, mx::v16f (&acc)[4][BN / 128]) {
    using T = Tile<BN, BK>;
    constexpr int TN = T::TN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int lr = lane & 31;
    const int h = lane >> 5;
    const int key = swz_key<T::CPR>(lr);
    const uint8_t* la = cur + (wm * 128 + lr) * T::ROWB;
    const uint8_t* lw = cur + T::A_BYTES + (wn * (BN / 4) + lr) * T::ROWB;
    const uint8_t* lsa = cur + T::A_BYTES + T::W_BYTES + (wm * 128 + lr) * T::SCB;
    const uint8_t* lsw = cur + T::A_BYTES + T::W_BYTES + BM * T::SCB + (wn * (BN / 4) + lr) * T::SCB;
    uint32_t sa[4], sb[TN];
#pragma unroll
    for (int i = 0; i < 4; ++i) sa[i] = scale_word<T::SCB>(lsa + i * 32 * T::SCB, h);
#pragma unroll
    for (int j = 0; j < TN; ++j) sb[j] = scale_word<T::SCB>(lsw + j * 32 * T::SCB, h);
#pragma unroll
    for (int ks = 0; ks < T::KS; ++ks) {
        const int koff = ((2 * ks + h) ^ key) << 4;
        uint4 af[4], bf[TN];
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = *reinterpret_cast<const uint4*>(la + koff + i * 32 * T::ROWB);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const uint4*>(lw + koff + j * 32 * T::ROWB);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if (ks == 0) acc[i][j] = mfma32<0>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
                if (ks == 1) acc[i][j] = mfma32<1>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
                if (ks == 2) acc[i][j] = mfma32<2>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
                if (ks == 3) acc[i][j] = mfma32<3>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
            }
    }
}

template <int BN, int BK, int NSTAGE>
__global__ __launch_bounds__(NTHREADS, 1) void gemm2_kernel(G2Args g) {
    using T = Tile<BN, BK>;
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
    const int wm = wave >> 2, wn = wave & 3;
    const int lr = lane & 31;
    const int h = lane >> 5;
    const int nsteps = g.Kp / BK;

    mx::v16f acc[4][TN];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

#pragma unroll
    for (int s = 0; s < NSTAGE - 1; ++s)
        if (s < nsteps) issue_stage<BN, BK>(g, ring + s * T::STAGE, m0, n0, s * BK);

    for (int it0 = 0; it0 < nsteps; it0 += NSTAGE) {
#pragma unroll
        for (int s = 0; s < NSTAGE; ++s) {
            const int it = it0 + s;
            if (it < nsteps) {
                // this wave's copies of step it have landed (those of the
                // NSTAGE-2 later steps may still be in flight) and its LDS
                // reads of step it-1 are done; after the barrier every wave's
                if (it + NSTAGE - 2 < nsteps)
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 2) * T::COPIES) : "memory");
                else
                    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                // refill the stage step it-1 used
                if (it + NSTAGE - 1 < nsteps)
                    issue_stage<BN, BK>(g, ring + ((s + NSTAGE - 1) % NSTAGE) * T::STAGE, m0, n0,
                                        (it + NSTAGE - 1) * BK);
                mfma_step<BN, BK>(ring + s * T::STAGE, acc);
            }
        }
    }

#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) mx::pin(acc[i][j]);
    // accumulator element e of lane l: row 8*(e/4) + 4*(l/32) + e%4, column l%32
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * (BN / 4) + j * 32 + lr;
            if (col >= g.N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (row < g.M) g.y[(int64_t)row * g.N + col] = acc[i][j][e];
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
// The 256 x 256 tile pays off when the grid fills at least half the CUs
// (measured on MI355X: 4096 x 4096 x 2048 in 29.8 us against 36.9 us for the
// 128 x 128 register-staged GEMM; 1024 x 4096 x 2048, 64 tiles, is faster there).
bool lin_pq_gemm2_supported(int M, int N, int Kp) {
    const int64_t tiles = (int64_t)((M + BM - 1) / BM) * ((N + 255) / 256);
    return M > 16 && N > 0 && Kp >= 256 && (Kp % 256) == 0 && tiles >= 128;
}

template <int BN, int BK, int NSTAGE>
int launch_gemm2(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc, float* y, int M, int N,
                 int Kp, hipStream_t st) {
    MXH_REQUIRE(Kp % BK == 0, "lin_pq_gemm2: Kp=%d is not a multiple of %d", Kp, BK);
    G2Args g{xq, xsc, wp, wsc, y, M, N, Kp, 0, 0, 0, 0, 0, 0};
    g.tiles_m = (M + BM - 1) / BM;
    g.tiles_n = (N + BN - 1) / BN;
    xcd_blocks(g);
    hipLaunchKernelGGL((gemm2_kernel<BN, BK, NSTAGE>), dim3(8 * g.per_xcd), dim3(NTHREADS), 0, st, g);
    return launch_status("lin_pq_gemm2");
}

int lin_pq_gemm2(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc, float* y,
                 int M, int N, int Kp, hipStream_t st) {
    MXH_REQUIRE(((uintptr_t)xq & 15) == 0 && ((uintptr_t)wp & 15) == 0,
                "lin_pq: packed operands must be 16-byte aligned");
    MXH_REQUIRE(((uintptr_t)xsc & 3) == 0 && ((uintptr_t)wsc & 3) == 0,
                "lin_pq: scale rows must be 4-byte aligned");
    return launch_gemm2<256, 256, 2>(xq, xsc, wp, wsc, y, M, N, Kp, st);
}
}  // namespace mxh
