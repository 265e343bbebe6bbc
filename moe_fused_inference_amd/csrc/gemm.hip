// gemm.hip -- block-scaled MXFP4 x MXFP4 GEMM (fp32 out) on CDNA4 MFMA.
//
// y (M, N) = A (M, Kp) * W (N, Kp)^T with both operands packed E2M1 rows and
// E8M0 32-block scales -- the lin_pq contract (src/ext/mxfp4_decode.cu:135-170)
// for M > 16.  The reference runs one m16n8k64 per warp per 64-K step with a
// serial, un-pipelined K loop; this kernel is designed for gfx950 instead:
//
// * Workgroup tile 128x128, 4 waves in 2x2, each wave 64x64 = 2x2
//   v_mfma_scale_f32_32x32x64_f8f6f4 accumulators (64 fp32 VGPRs).
// * K step 256: each operand tile is 128 rows x 128 B, i.e. exactly one 128-B
//   line per row per step; eight consecutive lanes read one row (coalesced).
// * LDS double buffer (2 x 38 KB): global loads of step k+1 are in flight
//   while step k's MFMAs run; rows are padded to 144 B so the ds_read_b128
//   operand fetches of 8 consecutive lanes hit distinct banks.
// * Scales: a lane needs block (2*ks + l/32) of its row for K-step ks; the 8
//   scale bytes of the row are loaded once per step and permuted (v_perm_b32)
//   so that op_sel = ks selects the right byte -- no per-step scale loads.
#include "mx_device.h"
#include "mx_host.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 256;
constexpr int ROWB = BK / 2;        // 128 data bytes per row per step
constexpr int LDSROW = ROWB + 16;   // padded LDS row
constexpr int SCB = BK / 32;        // 8 scale bytes per row per step
constexpr int TILE_BYTES = BM * LDSROW;
constexpr int BUF_BYTES = 2 * TILE_BYTES + 2 * BM * SCB;  // A, W data + A, W scales

template <int OP>
__device__ __forceinline__ mx::v16f mfma32(uint4 a, uint4 b, mx::v16f c, uint32_t sa, uint32_t sb) {
    mx::v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    mx::v8i bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 4, 4, OP, (int)sa, OP, (int)sb);
}

struct GemmArgs {
    const uint8_t* aq;
    const uint8_t* as;
    const uint8_t* wp;
    const uint8_t* ws;
    float* y;
    int M, N, Kp;
};

// Global -> registers for one K step: 4 x 16 B of A and 4 x 16 B of W per
// thread, plus 8 scale bytes of one row (threads 0..127: A, 128..255: W).
struct StageRegs {
    uint4 a[4];
    uint4 w[4];
    uint2 sc;
};

__device__ __forceinline__ void load_stage(StageRegs& r, const GemmArgs& g, int m0, int n0, int k0) {
    const int tid = threadIdx.x;
    const int nch = g.Kp >> 5;
    const int kb0 = k0 >> 5;            // first 32-block of this step
    const int cbytes = g.Kp >> 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid + 256 * i;
        const int row = idx >> 3;
        const int ch = idx & 7;          // 16-byte chunk = one 32-block
        const int blk = kb0 + ch;
        const bool kok = blk < nch;
        const int ar = min(m0 + row, g.M - 1);
        const int wr = min(n0 + row, g.N - 1);
        const int64_t off = (int64_t)(k0 >> 1) + ch * 16;
        r.a[i] = kok ? *reinterpret_cast<const uint4*>(g.aq + (int64_t)ar * cbytes + off) : make_uint4(0, 0, 0, 0);
        r.w[i] = kok ? *reinterpret_cast<const uint4*>(g.wp + (int64_t)wr * cbytes + off) : make_uint4(0, 0, 0, 0);
    }
    const int row = tid & 127;
    const bool isw = tid >= 128;
    const int rr = isw ? min(n0 + row, g.N - 1) : min(m0 + row, g.M - 1);
    const uint8_t* sp = (isw ? g.ws : g.as) + (int64_t)rr * nch + kb0;
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
        const int idx = tid + 256 * i;
        const int row = idx >> 3;
        const int ch = idx & 7;
        *reinterpret_cast<uint4*>(la + row * LDSROW + ch * 16) = r.a[i];
        *reinterpret_cast<uint4*>(lw + row * LDSROW + ch * 16) = r.w[i];
    }
    const int row = tid & 127;
    uint8_t* sdst = (tid >= 128 ? lsw : lsa) + row * SCB;
    *reinterpret_cast<uint2*>(sdst) = r.sc;
}

// Scale word for K-steps 0..3 of this lane: byte ks = block 2*ks + h.
__device__ __forceinline__ uint32_t scale_word(const uint8_t* srow, int h) {
    const uint2 v = *reinterpret_cast<const uint2*>(srow);
    return __builtin_amdgcn_perm(v.y, v.x, h ? 0x07050301u : 0x06040200u);
}

__global__ __launch_bounds__(256, 2) void gemm_mxfp4_kernel(GemmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int nsteps = (g.Kp + BK - 1) / BK;
    const int lr = lane & 31;
    const int h = lane >> 5;

    mx::v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    StageRegs st;
    load_stage(st, g, m0, n0, 0);
    store_stage(st, smem);
    __syncthreads();

    for (int it = 0; it < nsteps; ++it) {
        uint8_t* cur = smem + (it & 1) * BUF_BYTES;
        const bool more = it + 1 < nsteps;
        if (more) load_stage(st, g, m0, n0, (it + 1) * BK);

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
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (ks == 0) acc[i][j] = mfma32<0>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
                    if (ks == 1) acc[i][j] = mfma32<1>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
                    if (ks == 2) acc[i][j] = mfma32<2>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
                    if (ks == 3) acc[i][j] = mfma32<3>(af[i], bf[j], acc[i][j], sa[i], sb[j]);
                }
        }
        if (more) store_stage(st, smem + ((it + 1) & 1) * BUF_BYTES);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) mx::pin(acc[i][j]);
    // accumulator element e of lane l: row 8*(e/4) + 4*(l/32) + e%4, column l%32
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + lr;
            if (col >= g.N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (row < g.M) g.y[(int64_t)row * g.N + col] = acc[i][j][e];
            }
        }
}

}  // namespace

namespace mxh {
bool lin_pq_gemm_supported(int M, int N, int Kp) {
    // 16-byte row alignment of the packed operands (Kp/2 multiple of 16)
    return M > 0 && N > 0 && (Kp % 32) == 0;
}

int lin_pq_gemm(const uint8_t* xq, const uint8_t* xsc, const uint8_t* wp, const uint8_t* wsc, float* y,
                int M, int N, int Kp, hipStream_t st) {
    MXH_REQUIRE(((uintptr_t)xq & 15) == 0 && ((uintptr_t)wp & 15) == 0,
                "lin_pq: packed operands must be 16-byte aligned");
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_mxfp4_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 2 * BUF_BYTES);
        MXH_REQUIRE(e == hipSuccess, "lin_pq: cannot reserve %d B of LDS: %s", 2 * BUF_BYTES, hipGetErrorString(e));
        attr_set = true;
    }
    GemmArgs g{xq, xsc, wp, wsc, y, M, N, Kp};
    dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    hipLaunchKernelGGL(gemm_mxfp4_kernel, grid, dim3(256), 2 * BUF_BYTES, st, g);
    return launch_status("lin_pq_gemm");
}
}  // namespace mxh
