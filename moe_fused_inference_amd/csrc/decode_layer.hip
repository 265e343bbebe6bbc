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
// Workgroups are dispatched in index order, so every gate/up workgroup is
// resident or finished before any down workgroup waits: the wait cannot
// deadlock.  It is still bounded (kSpinLimit polls); on expiry the kernel sets
// an error flag, skips its work and exits normally.  The last down workgroup
// to finish resets the counters, so consecutive launches (or graph replays)
// need no host-side reset.
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

constexpr int kSpinLimit = 1 << 22;   // polls of the arrival counter (~0.2 s)
constexpr int kTerms = 3;             // E4M3 terms per activation value

struct LayerArgs {
    const uint16_t* x;        // (H) bf16
    const uint8_t* gate_wp;   // expert e at + e*gate_stride: (Mi, H/2)
    const uint8_t* gate_ws;   //                               (Mi, H/32)
    const uint8_t* up_wp;
    const uint8_t* up_ws;
    const uint8_t* down_wp;   // (H, Mi/2)
    const uint8_t* down_ws;   // (H, Mi/32)
    int64_t wp_stride_gu, ws_stride_gu;   // bytes between experts (gate/up)
    int64_t wp_stride_dn, ws_stride_dn;   // bytes between experts (down)
    const int32_t* ids_dev;   // (E) expert ids in device memory, or null
    const float* w_dev;       // (E) combine weights in device memory, or null
    int32_t ids[8];           // by-value ids when ids_dev is null
    float w[8];               // by-value weights when w_dev is null
    int E, H, Mi;
    float* out;               // (H) fp32 moe output
    uint16_t* resid;          // (H) bf16 x + bf16(out), or null
    uint8_t* hs8;             // workspace: (E, kTerms, Mi) E4M3 terms of h
    uint8_t* hsc;             // workspace: (E, kTerms, Mi/32) scale codes
    int* sync;                // workspace: [0] arrivals, [1] departures, [2] error
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
// aligned) into kTerms E4M3 terms.  Writes 8 bytes per term to dst8[t] and, on
// the quad's first lane, the term's scale code to dsc[t].
__device__ __forceinline__ void split8(float v[8], uint8_t* const dst8[kTerms], uint8_t* const dsc[kTerms],
                                       bool writer) {
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
            // residual for the next term: value - decode(code)*scale (exact)
            typedef float v2f __attribute__((ext_vector_type(2)));
            v2f d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word[h], sc, false);
            v2f d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word[h], sc, true);
            v[4 * h + 0] -= d0[0];
            v[4 * h + 1] -= d0[1];
            v[4 * h + 2] -= d1[0];
            v[4 * h + 3] -= d1[1];
        }
        *reinterpret_cast<uint2*>(dst8[t]) = make_uint2(word[0], word[1]);
        if (writer) *dsc[t] = (uint8_t)code;
    }
}

// FP8-A operand of one MFMA K-step for lane (r = term row, g) when the 4 lane
// groups' 32-blocks of this step are phys_blk[0..3] (B lane group gb holds
// block phys_blk[gb]): bytes 0..15 <- logical K 16g..16g+15 (B group g/2,
// elements 16*(g%2)..), bytes 16..31 <- logical K 64+16g.. (B group 2+g/2).
__device__ __forceinline__ mx::v8i fp8_operand(const uint8_t* row8, int blk_lo, int blk_hi, int g) {
    const uint4 lo = *reinterpret_cast<const uint4*>(row8 + blk_lo * 32 + 16 * (g & 1));
    const uint4 hi = *reinterpret_cast<const uint4*>(row8 + blk_hi * 32 + 16 * (g & 1));
    mx::v8i a = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    return a;
}

__device__ __forceinline__ void wait_arrivals(const LayerArgs& a, int target, int* s_abort) {
    if (threadIdx.x == 0) {
        int spins = 0;
        int ok = 1;
        while (__hip_atomic_load(&a.sync[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(2);
            if (++spins >= kSpinLimit) {
                ok = 0;
                break;
            }
        }
        if (ok) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // pairs with the gate/up release
        } else {
            __hip_atomic_store(&a.sync[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *s_abort = !ok;
    }
    __syncthreads();
}

template <bool DEV_IDS>
__global__ __launch_bounds__(256) void decode_layer_kernel(LayerArgs a) {
    __shared__ __align__(16) uint8_t s_x8[kTerms][2048];   // E4M3 terms of x (H <= 2048)
    __shared__ uint8_t s_xsc[kTerms][64];
    __shared__ float s_red[4][4][16];
    __shared__ float s_h[2][32];
    __shared__ int s_abort;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int nblk_mi = a.Mi >> 5;
    const int nA = a.E * nblk_mi;
    const int bid = blockIdx.x;

    if (bid < nA) {
        // ================================================= gate / up
        const int s = bid % a.E;
        const int jb = bid / a.E;
        const int j0 = jb * 32;
        const int e = DEV_IDS ? a.ids_dev[s] : a.ids[s];
        const int H = a.H;
        const int hb = H >> 5;                  // 32-blocks per row (64)
        const int bpw = hb >> 2;                // blocks per wave (16)
        const uint8_t* gw = a.gate_wp + (int64_t)e * a.wp_stride_gu;
        const uint8_t* gs = a.gate_ws + (int64_t)e * a.ws_stride_gu;
        const uint8_t* uw = a.up_wp + (int64_t)e * a.wp_stride_gu;
        const uint8_t* us = a.up_ws + (int64_t)e * a.ws_stride_gu;

        // weights: 4 row groups (gate lo/hi, up lo/hi) x sa K-steps; lane
        // group g owns blocks bpw*wave + sa*g .. +sa-1 of its row (contiguous)
        const int sa = bpw >> 2;                // K-steps per wave (H/512, <= 4)
        uint4 bq[4][4];
        uint32_t bsc[4][4];
        const int blk0 = bpw * wave + sa * g;
#pragma unroll
        for (int G = 0; G < 4; ++G) {
            const int row = j0 + 16 * (G & 1) + r;
            const uint8_t* wrow = ((G < 2) ? gw : uw) + (int64_t)row * (H >> 1);
            const uint8_t* srow = ((G < 2) ? gs : us) + (int64_t)row * hb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool ok = i < sa;
                bq[G][i] = ok ? *reinterpret_cast<const uint4*>(wrow + (blk0 + i) * 16) : make_uint4(0, 0, 0, 0);
                bsc[G][i] = ok ? (uint32_t)srow[blk0 + i] : 127u;
            }
        }

        // x -> three E4M3 terms in LDS (whole row; 8 values per thread)
        {
            const int k0 = threadIdx.x * 8;
            float v[8];
            if (k0 < H) {
                const uint4 q = *reinterpret_cast<const uint4*>(a.x + k0);
                const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[2 * i] = mx::bf16_to_f32((uint16_t)(w4[i] & 0xFFFFu));
                    v[2 * i + 1] = mx::bf16_to_f32((uint16_t)(w4[i] >> 16));
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = 0.0f;
            }
            uint8_t* d8[kTerms] = {&s_x8[0][k0 & 2047], &s_x8[1][k0 & 2047], &s_x8[2][k0 & 2047]};
            uint8_t* dsc[kTerms] = {&s_xsc[0][(k0 >> 5) & 63], &s_xsc[1][(k0 >> 5) & 63], &s_xsc[2][(k0 >> 5) & 63]};
            if (k0 < H) split8(v, d8, dsc, (threadIdx.x & 3) == 0);
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
                av = fp8_operand(s_x8[r], base + sa * (g >> 1), base + sa * (2 + (g >> 1)), g);
                asc = s_xsc[r][base + sa * g];
            }
#pragma unroll
            for (int G = 0; G < 4; ++G) acc[G] = mx::mfma16_fp8a_fp4b(av, bq[G][i], acc[G], asc, bsc[G][i]);
        }
        // rows 0..2 of D (the three terms) are elements 0..2 of lanes 0..15
        if (lane < 16) {
#pragma unroll
            for (int G = 0; G < 4; ++G) s_red[wave][G][lane] = acc[G][0] + acc[G][1] + acc[G][2];
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            const int G = threadIdx.x >> 4;   // 0,1 gate halves; 2,3 up halves
            const int n = threadIdx.x & 15;
            const float v = s_red[0][G][n] + s_red[1][G][n] + s_red[2][G][n] + s_red[3][G][n];
            s_h[G >> 1][16 * (G & 1) + n] = v;
        }
        __syncthreads();
        // h = silu(g) * u for the 32 rows, split into E4M3 terms -> workspace
        if (threadIdx.x < 4) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int j = threadIdx.x * 8 + i;
                v[i] = mx::silu_mul(s_h[0][j], s_h[1][j]);
            }
            uint8_t* d8[kTerms];
            uint8_t* dsc[kTerms];
#pragma unroll
            for (int t = 0; t < kTerms; ++t) {
                d8[t] = a.hs8 + ((int64_t)s * kTerms + t) * a.Mi + j0 + threadIdx.x * 8;
                dsc[t] = a.hsc + ((int64_t)s * kTerms + t) * nblk_mi + jb;
            }
            split8(v, d8, dsc, threadIdx.x == 0);
        }
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(&a.sync[0], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // ===================================================== down + combine
    const int cb = bid - nA;
    const int c0 = cb * 16;
    const int Mi = a.Mi;
    const int kb = Mi >> 5;          // 32-blocks per down row (24)
    const int steps = (kb + 3) >> 2; // MFMA K-steps (6)
    // wave handles slots 2*wave, 2*wave+1; lane group g owns blocks
    // g*steps .. g*steps+steps-1 of its row
    uint4 bq[2][8];
    uint32_t bsc[2][8];
    int slot[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        slot[q] = 2 * wave + q;
        const bool live = slot[q] < a.E;
        const int e = live ? (DEV_IDS ? a.ids_dev[slot[q]] : a.ids[slot[q]]) : 0;
        const uint8_t* wrow = a.down_wp + (int64_t)e * a.wp_stride_dn + (int64_t)(c0 + r) * (Mi >> 1);
        const uint8_t* srow = a.down_ws + (int64_t)e * a.ws_stride_dn + (int64_t)(c0 + r) * kb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int blk = g * steps + i;
            const bool ok = live && i < steps && blk < kb;
            bq[q][i] = ok ? *reinterpret_cast<const uint4*>(wrow + blk * 16) : make_uint4(0, 0, 0, 0);
            bsc[q][i] = ok ? (uint32_t)srow[blk] : 127u;
        }
    }

    wait_arrivals(a, nA, &s_abort);
    const bool abort = s_abort != 0;

    float part = 0.0f;  // this lane's (lane < 16) partial combine over its slots
    if (!abort) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            if (slot[q] >= a.E) continue;
            mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
            const uint8_t* h8 = a.hs8 + ((int64_t)slot[q] * kTerms + (r < kTerms ? r : 0)) * Mi;
            const uint8_t* hsc = a.hsc + ((int64_t)slot[q] * kTerms + (r < kTerms ? r : 0)) * kb;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (i >= steps) break;
                mx::v8i av = {0, 0, 0, 0, 0, 0, 0, 0};
                uint32_t asc = 127u;
                // step i: B lane group gb holds block gb*steps + i
                const int blo = (g >> 1) * steps + i;
                const int bhi = (2 + (g >> 1)) * steps + i;
                const int bown = g * steps + i;
                if (r < kTerms) {
                    if (blo < kb) {
                        const uint4 lo = *reinterpret_cast<const uint4*>(h8 + blo * 32 + 16 * (g & 1));
                        av[0] = (int)lo.x; av[1] = (int)lo.y; av[2] = (int)lo.z; av[3] = (int)lo.w;
                    }
                    if (bhi < kb) {
                        const uint4 hi = *reinterpret_cast<const uint4*>(h8 + bhi * 32 + 16 * (g & 1));
                        av[4] = (int)hi.x; av[5] = (int)hi.y; av[6] = (int)hi.z; av[7] = (int)hi.w;
                    }
                    if (bown < kb) asc = hsc[bown];
                }
                acc = mx::mfma16_fp8a_fp4b(av, bq[q][i], acc, asc, bsc[q][i]);
            }
            const float we = DEV_IDS && a.w_dev ? a.w_dev[slot[q]] : a.w[slot[q]];
            part = fmaf(we, acc[0] + acc[1] + acc[2], part);
        }
    }
    if (lane < 16) s_red[wave][0][lane] = part;
    __syncthreads();
    if (!abort && threadIdx.x < 16) {
        const int c = c0 + threadIdx.x;
        const float y = s_red[0][0][threadIdx.x] + s_red[1][0][threadIdx.x] + s_red[2][0][threadIdx.x] +
                        s_red[3][0][threadIdx.x];
        a.out[c] = y;
        if (a.resid) {
            // runtime/model_runner_v2.py:208: x = x + moe.bfloat16() in bf16
            const float yb = mx::bf16_to_f32(mx::f32_to_bf16_rne(y));
            a.resid[c] = mx::f32_to_bf16_rne(mx::bf16_to_f32(a.x[c]) + yb);
        }
    }
    // departure; the last down workgroup resets the counters for the next launch
    if (threadIdx.x == 0) {
        const int nB = gridDim.x - nA;
        const int old = __hip_atomic_fetch_add(&a.sync[1], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (old == nB - 1) {
            __hip_atomic_store(&a.sync[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.sync[1], 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

__global__ void reset_sync_kernel(int* sync) {
    if (threadIdx.x < 4) sync[threadIdx.x] = 0;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

extern "C" size_t mxfp4_decode_layer_workspace_size(int E, int Mi) {
    if (E <= 0 || Mi <= 0) return 0;
    return 256 + align256((size_t)E * kTerms * Mi) + align256((size_t)E * kTerms * (Mi / 32));
}

extern "C" int mxfp4_decode_layer_reset(void* workspace, void* stream) {
    MXH_REQUIRE(workspace, "decode_layer_reset: null workspace");
    hipLaunchKernelGGL(reset_sync_kernel, dim3(1), dim3(64), 0, mxh::as_stream(stream),
                       static_cast<int*>(workspace));
    return mxh::launch_status("decode_layer_reset");
}

extern "C" int mxfp4_decode_layer_status(const void* workspace, int* error_flag) {
    MXH_REQUIRE(workspace && error_flag, "decode_layer_status: null pointer");
    int host[4];
    hipError_t e = hipMemcpy(host, workspace, sizeof host, hipMemcpyDeviceToHost);
    MXH_REQUIRE(e == hipSuccess, "decode_layer_status: %s", hipGetErrorString(e));
    *error_flag = host[2];
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
    MXH_REQUIRE(E >= 1 && E <= 8, "moe_decode_layer: E=%d must be in [1, 8]", E);
    MXH_REQUIRE(H % 512 == 0 && H >= 512 && H <= 2048, "moe_decode_layer: H=%d must be a multiple of 512 in [512, 2048]", H);
    MXH_REQUIRE(Mi % 32 == 0 && Mi >= 32 && Mi <= 32 * 8 * 4, "moe_decode_layer: Mi=%d must be a multiple of 32 <= 1024", Mi);
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
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    a.sync = reinterpret_cast<int*>(ws);
    a.hs8 = ws + 256;
    a.hsc = a.hs8 + align256((size_t)E * kTerms * Mi);
    const int nA = E * (Mi / 32);
    const int nB = H / 16;
    if (ids_dev)
        hipLaunchKernelGGL(decode_layer_kernel<true>, dim3(nA + nB), dim3(256), 0, mxh::as_stream(stream), a);
    else
        hipLaunchKernelGGL(decode_layer_kernel<false>, dim3(nA + nB), dim3(256), 0, mxh::as_stream(stream), a);
    return mxh::launch_status("moe_decode_layer");
}
