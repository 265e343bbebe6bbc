// decode_stack.hip -- a run of consecutive decode MoE layers for one token in
// one launch (batch 1).
//
// Computes, for layers l = 0 .. L-1 of a stack,
//     y_l     = sum_s w[l][s] * down_e(silu(gate_e(x_l)) * up_e(x_l)),  e = ids[l][s]
//     x_{l+1} = bf16(x_l + bf16(y_l))
// -- the reference's per-layer MoE step (runtime/model_runner_v2.py:185-208,
// kernels src/ext/mxfp4_decode.cu:24-50,177-299) applied layer after layer,
// on un-quantized bf16 activations in fp32 like the one-layer kernel
// (decode_layer.hip).  The routing of every layer (ids, w) is an input, so
// the kernel can fetch layer l+1's expert weights while layer l is still
// being computed: the launch streams weights at HBM rate instead of paying a
// launch and a cold weight burst per layer.
//
// Workgroups keep one role for the whole launch (the one-layer kernel's
// split):
//   [0, nA)        gate/up tile (slot s, 32 intermediate rows) of every layer:
//                  wait for x_l, h = silu(g)*u, publish h_l (E4M3 terms);
//   [nA, nA+nB)    down + combine, 32 output columns of every layer: wait for
//                  h_l, y, x_{l+1} = bf16(x_l + bf16(y)), publish x_{l+1}.
// A gate/up workgroup issues layer l+1's weight loads right after its layer-l
// MFMAs, a down workgroup right after its layer-l MFMAs, so both weight
// streams run under the other phase and the hand-offs.  With STRICT the loads
// of layer l are issued only once x_l is complete (down workgroups then wait
// for x_l as well): the timing of a model whose routing depends on x_l.
//
// Hand-offs.  As in the one-layer kernel a published 32-bit word is its own
// flag (kEmpty = not yet): h words carry three E4M3 term bytes (+ the terms'
// codes in byte 3 of a record's first three words), x words carry the bf16
// value in their low half (high half 0, so never kEmpty).  Producers store with
// agent-scope atomic stores; consumers poll with agent-scope loads.  Each
// value has three buffers, used round robin by a per-workgroup layer count
// ("memo", read at entry, + L stored at exit; all workgroups agree on it):
// layer count c publishes into buffer c%3 and then empties its words of
// buffer (c-1)%3, which is published into again at layer c+2.  That is safe:
// the readers of (c-1)%3 were the consumers of layer c-1, which the producer
// has already waited for (a gate/up workgroup at layer c has all of x_c,
// which the down workgroups publish after reading h_{c-1}; a down workgroup
// at layer c has all of h_c, which the gate/up workgroups publish after
// reading x_c).  Before each publish a producer waits for its earlier stores
// (s_waitcnt vmcnt(0)), so the empties of layer c are visible before anything
// of layer c+1 is, hence before any consumer polls (c+2)%3 -- a layer after
// they were issued, so the wait is normally free.  No reset is needed between
// launches.
//
// Co-residency.  The grid (E*Mi/32 + H/32 = 256 workgroups at the headline
// shape) must be resident at once: every workgroup waits on others of every
// layer.  Each workgroup takes more than half of a CU's LDS, so it has a CU
// to itself, and the host refuses a grid larger than the CU count.  (With two
// workgroups on a CU -- a gate/up and a down workgroup -- the down
// workgroup's polls were seen to miss a published word for up to a second
// while its CU neighbour was polling, which stalled the whole chain.)  Every
// wait is bounded (kSpinLimit polls); on expiry, or when another workgroup
// has set the error flag, a thread stops waiting, the results are garbage and
// the flag stays set until the workspace is reset.
#include "decode_common.h"
#include "mx_host.h"

namespace {

using namespace dl;

// workspace layout (bytes)
constexpr int kCfgOff = 0;            // int32 config word written by reset
constexpr int kErrOff = 256;          // int32 error flag
constexpr int kMemoOff = 1024;        // int32 layer count per workgroup
constexpr int kMaxWg = 768;
constexpr int kBufOff = kMemoOff + 4 * kMaxWg;   // h buffers, then x buffers (uint32 words)
constexpr int kNBuf = 3;              // buffers per value, used round robin by layer count

struct StackLayer {
    const uint8_t* wp[3];   // gate, up, down packed data of the layer's experts (stacked)
    const uint8_t* ws[3];   // their E8M0 scales
};

struct StackArgs {
    const StackLayer* layers;   // (L) in device memory
    const int32_t* ids;         // (L, E) expert ids
    const float* w;             // (L, E) combine weights
    const uint16_t* x0;         // (H) bf16 input of layer 0
    uint16_t* x_out;            // (H) bf16 x_L
    uint16_t* x_all;            // optional (L, H) bf16 x_{l+1}
    float* y_all;               // optional (L, H) fp32 y_l
    int64_t wp_stride_gu, ws_stride_gu;   // bytes between experts (gate/up)
    int64_t wp_stride_dn, ws_stride_dn;   // bytes between experts (down)
    int n_layers, n_experts, E, H, Mi;
    int cfg;                    // expected workspace config word
    int hwords;                 // words between consecutive h buffers
    int xwords;                 // words between consecutive x buffers
    uint8_t* ws;
};

__host__ __device__ constexpr int stack_cfg(int E, int H, int Mi) {
    return 0x5B000000 | (E << 16) | ((H / 512) << 12) | (Mi / 32);
}

union Smem {
    struct {                                       // gate/up workgroups
        uint4 zero[2];
        uint8_t x8[kTerms][2048];
        uint8_t xsc[kTerms][64];
        float red[4][4][16];
    } a;
    struct {                                       // down workgroups
        uint4 zero[2];
        uint32_t code127[4];
        uint8_t h8[kMaxE * kTerms * 1024];
        uint32_t hsc[kMaxE * 32];
        float red[4][32];
    } b;
    uint8_t one_per_cu[84 * 1024];                 // more than half of a CU's LDS: one workgroup per CU
};

__device__ __forceinline__ void set_error(const StackArgs& a) {
    __hip_atomic_store(reinterpret_cast<int*>(a.ws + kErrOff), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool error_set(const StackArgs& a) {
    return __hip_atomic_load(reinterpret_cast<const int*>(a.ws + kErrOff), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Workgroup barrier for LDS only: waits for this wave's LDS operations, not
// for its outstanding global loads (__syncthreads' release fence would wait
// for the next layer's weight prefetch).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Waits for every outstanding global memory operation of this wave: makes
// the agent-scope stores issued so far visible before any later store.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Bounded poll of N 16-byte groups at byte offsets off[i] of buffer rs until
// none of their words is kEmpty; every round reloads all groups with the
// agent-scope cache policy (one round trip per check: a one-word probe
// before the full reload would cost a second one).  `live` false (an earlier
// wait failed): one load, no wait.  Returns false on expiry or when the error
// flag is set.
template <int N>
__device__ __forceinline__ bool poll_groups(const StackArgs& a, __amdgpu_buffer_rsrc_t rs,
                                            const int (&off)[N], v4u (&v)[N], bool live) {
    int spins = 0;
    while (true) {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[i], 0, 16);
        if (!live) return false;
        bool pending = false;
#pragma unroll
        for (int i = 0; i < N; ++i) pending |= (v[i].x == kEmpty) | (v[i].y == kEmpty) | (v[i].z == kEmpty) | (v[i].w == kEmpty);
        if (__builtin_amdgcn_ballot_w64(pending) == 0) return true;   // the wave polls as one
        if (++spins >= kSpinLimit || ((spins & 255) == 0 && error_set(a))) return false;
        __builtin_amdgcn_s_sleep(1);
        asm volatile("" ::: "memory");   // the words may change: reload them next round
    }
}

// x_l (H <= 2048 bf16) from the x buffer: thread t waits for words 8t..8t+7
// and returns their values packed as 8 bf16 (threads past H read zeros).
__device__ __forceinline__ bool wait_x(const StackArgs& a, const uint32_t* xb, uint4& xq, bool live) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(xb), (short)0,
                                                                        a.H * 4, 0x00020000);
    const int t8 = min(8 * (int)threadIdx.x, a.H - 8);   // threads past H re-poll the last group
    const int off[2] = {t8 * 4, t8 * 4 + 16};
    v4u v[2];
    const bool ok = poll_groups<2>(a, rs, off, v, live);
    const bool in = 8 * (int)threadIdx.x < a.H;
    xq.x = in ? (v[0].x & 0xFFFFu) | (v[0].y << 16) : 0u;
    xq.y = in ? (v[0].z & 0xFFFFu) | (v[0].w << 16) : 0u;
    xq.z = in ? (v[1].x & 0xFFFFu) | (v[1].y << 16) : 0u;
    xq.w = in ? (v[1].z & 0xFFFFu) | (v[1].w << 16) : 0u;
    return ok;
}

template <bool STRICT, int MS>
__global__ __launch_bounds__(256, 1) void decode_stack_kernel(StackArgs a) {
    __shared__ __align__(16) Smem sm;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const int rr = r < kTerms ? r : 0;
    const int nblk_mi = a.Mi >> 5;
    const int nA = a.E * nblk_mi;
    const int bid = blockIdx.x;
    const int L = a.n_layers;
    const int E = a.E;
    const int H = a.H;
    int* memo = reinterpret_cast<int*>(a.ws + kMemoOff) + bid;
    const int c0 = __builtin_amdgcn_readfirstlane(*memo);   // uniform: buffer selects stay scalar
    const bool cfg_ok = *reinterpret_cast<const int*>(a.ws + kCfgOff) == a.cfg;
    if (!cfg_ok) {
        if (threadIdx.x == 0) set_error(a);
        return;
    }
    uint32_t* hbuf = reinterpret_cast<uint32_t*>(a.ws + kBufOff);
    uint32_t* xbuf = hbuf + kNBuf * a.hwords;
    bool live = true;   // this thread's waits have all succeeded

    if (bid < nA) {
        // ================================================= gate / up
        const int s = bid % E;
        const int jb = bid / E;
        const int j0 = jb * 32;
        const int hb = H >> 5;
        const int bpw = hb >> 2;
        const int sa = bpw >> 2;
        const int k0 = threadIdx.x * 8;
        const int blk0 = bpw * wave + sa * g;
        if (threadIdx.x < 2) sm.a.zero[threadIdx.x] = make_uint4(0, 0, 0, 0);

        uint4 bq[4][4];
        uint32_t bsc4[4];
        auto load_w = [&](int l) {
            int e = __builtin_amdgcn_readfirstlane(a.ids[l * E + s]);
            e = e < 0 ? 0 : (e >= a.n_experts ? a.n_experts - 1 : e);   // memory safety only
            const StackLayer* ly = a.layers + l;
            const uint8_t* gw = ly->wp[0] + (int64_t)e * a.wp_stride_gu;
            const uint8_t* gs = ly->ws[0] + (int64_t)e * a.ws_stride_gu;
            const uint8_t* uw = ly->wp[1] + (int64_t)e * a.wp_stride_gu;
            const uint8_t* us = ly->ws[1] + (int64_t)e * a.ws_stride_gu;
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
                const int d0 = blk0 & ~3;
                const uint32_t lo = *reinterpret_cast<const uint32_t*>(srow + d0);
                const uint32_t hi = *reinterpret_cast<const uint32_t*>(srow + min(d0 + 4, hb - 4));
                bsc4[G] = (uint32_t)((((uint64_t)hi << 32) | lo) >> (8 * (blk0 & 3)));
            }
        };
        if (!STRICT) load_w(0);

        const int64_t w_off = ((int64_t)s * nblk_mi + jb) * kRecWords + (lane & 31);
        for (int l = 0; l < L; ++l) {
            const int b = (c0 + l) % kNBuf;             // this layer's buffer
            const int bprev = (b + kNBuf - 1) % kNBuf;  // the previous layer's
            uint4 xq = make_uint4(0, 0, 0, 0);
            if (l == 0) {
                if (k0 < H) xq = *reinterpret_cast<const uint4*>(a.x0 + k0);
            } else {
                live = wait_x(a, xbuf + bprev * a.xwords, xq, live);
            }
            if (STRICT) load_w(l);

            // x_l -> three E4M3 terms in LDS
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
            lds_barrier();

            mx::v8i av[4];
            uint32_t asc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int base = bpw * wave + min(i, sa - 1);
                const bool ok = r < kTerms && i < sa;
                const uint4* plo = ok ? reinterpret_cast<const uint4*>(&sm.a.x8[rr][(base + sa * (g >> 1)) * 32 + 16 * (g & 1)])
                                      : &sm.a.zero[0];
                const uint4* phi = ok ? reinterpret_cast<const uint4*>(&sm.a.x8[rr][(base + sa * (2 + (g >> 1))) * 32 + 16 * (g & 1)])
                                      : &sm.a.zero[1];
                av[i] = cat8(*plo, *phi);
                const uint32_t c = sm.a.xsc[rr][base + sa * g];
                asc[i] = ok ? c : 127u;
            }
            mx::v4f acc[4];
#pragma unroll
            for (int G = 0; G < 4; ++G) acc[G] = (mx::v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int G = 0; G < 4; ++G)
                    acc[G] = mx::mfma16_fp8a_fp4b(av[i], bq[G][i], acc[G], asc[i], (bsc4[G] >> (8 * i)) & 0xFFu);
#pragma unroll
            for (int G = 0; G < 4; ++G) mx::pin(acc[G]);
            if (lane < 16) {
#pragma unroll
                for (int G = 0; G < 4; ++G) sm.a.red[wave][G][lane] = acc[G][0] + acc[G][1] + acc[G][2];
            }
            lds_barrier();
            if (wave == 0) {
                const int j = lane & 31;
                float gsum = 0.f, usum = 0.f;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    gsum += sm.a.red[w][j >> 4][j & 15];
                    usum += sm.a.red[w][2 + (j >> 4)][j & 15];
                }
                uint32_t codes;
                const uint32_t bytes = split32(mx::silu_mul(gsum, usum), codes);
                const uint32_t word = bytes | (j < kTerms ? ((codes >> (8 * j)) & 0xFFu) << 24 : 0u);
                wait_stores();   // the previous layer's empty-stores are visible before this publish
                if (lane < 32) {
                    __hip_atomic_store(hbuf + b * a.hwords + w_off, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    // empty this record in the previous layer's buffer (written
                    // again two layers on; its readers, the down workgroups of
                    // the previous layer, are done: x_l is complete)
                    __hip_atomic_store(hbuf + bprev * a.hwords + w_off, kEmpty, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            // The next layer's weights stream under the down phase.  Issued
            // after the publish: a burst of loads stalls the issuing wave
            // once the CU's memory queue is full.
            if (!STRICT && l + 1 < L) load_w(l + 1);
        }
        if (!live) set_error(a);
        if (threadIdx.x == 0) *memo = c0 + L;
        return;
    }

    // ===================================================== down + combine
    // 32 output columns: column blocks cq = 0, 1 of 16 (one MFMA tile each);
    // wave w owns slots 2w, 2w+1 of both blocks (the h operand of a slot is
    // shared by the two blocks)
    const int cb = bid - nA;
    const int c0c = cb * 32;
    const int Mi = a.Mi;
    const int kb = Mi >> 5;
    const int steps = (kb + 3) >> 2;
    if (threadIdx.x < 2) sm.b.zero[threadIdx.x] = make_uint4(0, 0, 0, 0);
    if (threadIdx.x == 2) sm.b.code127[0] = 0x7F7F7F7Fu;
    // x_l of this workgroup's 32 columns (threads 0..31): layer 0 from the
    // input, later layers from this workgroup's own previous result
    float xown = 0.0f;
    if (threadIdx.x < 32) xown = mx::bf16_to_f32(a.x0[c0c + threadIdx.x]);

    uint4 bq[2][2][MS];      // [slot q][column block cq][K step]
    uint32_t bsw[2][2][3];
    int slot[2];
    float wgt[2];
    auto load_w = [&](int l) {
        const StackLayer* ly = a.layers + l;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            slot[q] = 2 * wave + q;
            const int sl = slot[q] < E ? slot[q] : 0;
            int e = __builtin_amdgcn_readfirstlane(a.ids[l * E + sl]);
            e = e < 0 ? 0 : (e >= a.n_experts ? a.n_experts - 1 : e);
            wgt[q] = a.w[l * E + sl];
            const bool lv = slot[q] < E;
#pragma unroll
            for (int cq = 0; cq < 2; ++cq) {
                const int row = c0c + 16 * cq + r;
                const uint8_t* wrow = ly->wp[2] + (int64_t)e * a.wp_stride_dn + (int64_t)row * (Mi >> 1);
                const uint8_t* srow = ly->ws[2] + (int64_t)e * a.ws_stride_dn + (int64_t)row * kb;
#pragma unroll
                for (int i = 0; i < MS; ++i) {
                    const int blk = g * steps + i;
                    bq[q][cq][i] = ld_sel(reinterpret_cast<const uint4*>(wrow + min(blk, kb - 1) * 16),
                                          lv && i < steps && blk < kb, make_uint4(0, 0, 0, 0));
                }
                const int sb0 = (g * steps) & ~3;
                if ((kb & 3) == 0) {
#pragma unroll
                    for (int d = 0; d < 3; ++d)
                        bsw[q][cq][d] = *reinterpret_cast<const uint32_t*>(srow + min(sb0 + 4 * d, kb - 4));
                } else {
#pragma unroll
                    for (int d = 0; d < 3; ++d) {
                        uint32_t v = 0;
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int off = sb0 + 4 * d + b;
                            v |= ((lv && off < kb) ? (uint32_t)srow[off] : 127u) << (8 * b);
                        }
                        bsw[q][cq][d] = v;
                    }
                }
            }
        }
    };
    if (!STRICT) load_w(0);

    const int nwords = E * nblk_mi * kRecWords;
    constexpr int kGroups = (kMaxE * 4 * MS * kRecWords) / 2048;
    for (int l = 0; l < L; ++l) {
        const int b = (c0 + l) % kNBuf;
        const int bprev = (b + kNBuf - 1) % kNBuf;
        if (STRICT) {
            if (l > 0) {
                uint4 unused;
                live = wait_x(a, xbuf + bprev * a.xwords, unused, live);
            }
            load_w(l);
        }
        // h_l: poll all words, unpack term bytes and codes into LDS
        const uint32_t* cur = hbuf + b * a.hwords;
        {
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(cur), (short)0, nwords * 4, 0x00020000);
            int off[2 * kGroups];
#pragma unroll
            for (int k = 0; k < kGroups; ++k)
#pragma unroll
                for (int h = 0; h < 2; ++h) off[2 * k + h] = min(2048 * k + 8 * (int)threadIdx.x + 4 * h, nwords - 4) * 4;
            v4u v[2 * kGroups];
            live = poll_groups<2 * kGroups>(a, rs, off, v, live);
#pragma unroll
            for (int k = 0; k < kGroups; ++k) {
                const int wi = 2048 * k + 8 * (int)threadIdx.x;
                if (wi < nwords) {
                    const uint32_t wv[8] = {v[2 * k].x, v[2 * k].y, v[2 * k].z, v[2 * k].w,
                                            v[2 * k + 1].x, v[2 * k + 1].y, v[2 * k + 1].z, v[2 * k + 1].w};
                    const int rec = 64 * k + ((int)threadIdx.x >> 2);
#pragma unroll
                    for (int t = 0; t < kTerms; ++t) {
                        const uint32_t sel = 0x0C0C0000u | ((4u + t) << 8) | (uint32_t)t;
                        const uint32_t lo = __builtin_amdgcn_perm(wv[1], wv[0], sel) |
                                            (__builtin_amdgcn_perm(wv[3], wv[2], sel) << 16);
                        const uint32_t hi = __builtin_amdgcn_perm(wv[5], wv[4], sel) |
                                            (__builtin_amdgcn_perm(wv[7], wv[6], sel) << 16);
                        *reinterpret_cast<uint64_t*>(sm.b.h8 + (rec * kTerms + t) * 32 + 8 * (threadIdx.x & 3)) =
                            (uint64_t)lo | ((uint64_t)hi << 32);
                    }
                    if ((threadIdx.x & 3) == 0)
                        sm.b.hsc[rec] = (wv[0] >> 24) | ((wv[1] >> 24) << 8) | ((wv[2] >> 24) << 16);
                }
            }
        }
        lds_barrier();

        const int sb0 = (g * steps) & ~3;
        bool lv[2];
        const uint8_t* h8[2];
        const uint32_t* hsq[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            lv[q] = slot[q] < E;
            const int sl = lv[q] ? slot[q] : 0;
            h8[q] = sm.b.h8 + (sl * kb * kTerms + rr) * 32;
            hsq[q] = sm.b.hsc + sl * kb;
        }
        const float w0 = wgt[0], w1 = wgt[1];
        mx::v4f acc[2][2] = {{{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}, {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}}};
#pragma unroll
        for (int i = 0; i < MS; ++i) {
            const int blo = (g >> 1) * steps + i;
            const int bhi = (2 + (g >> 1)) * steps + i;
            const int bown = g * steps + i;
            const bool rok = r < kTerms && i < steps;
            const int bi = g * steps + i - sb0;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const bool ok = rok && lv[q];
                const uint4* plo = (ok && blo < kb) ? reinterpret_cast<const uint4*>(h8[q] + blo * (kTerms * 32) + 16 * (g & 1))
                                                    : &sm.b.zero[0];
                const uint4* phi = (ok && bhi < kb) ? reinterpret_cast<const uint4*>(h8[q] + bhi * (kTerms * 32) + 16 * (g & 1))
                                                    : &sm.b.zero[1];
                const uint32_t* pc = (ok && bown < kb) ? &hsq[q][bown] : &sm.b.code127[0];
                const mx::v8i av = cat8(*plo, *phi);
                const uint32_t asc = (*pc >> (8 * rr)) & 0xFFu;
#pragma unroll
                for (int cq = 0; cq < 2; ++cq) {
                    const uint32_t wd = bi < 4 ? bsw[q][cq][0] : (bi < 8 ? bsw[q][cq][1] : bsw[q][cq][2]);
                    acc[q][cq] = mx::mfma16_fp8a_fp4b(av, bq[q][cq][i], acc[q][cq], asc, (wd >> (8 * (bi & 3))) & 0xFFu);
                }
            }
        }
        float part[2] = {0.0f, 0.0f};
#pragma unroll
        for (int cq = 0; cq < 2; ++cq) {
#pragma unroll
            for (int q = 0; q < 2; ++q) mx::pin(acc[q][cq]);
            if (lv[0]) part[cq] = fmaf(w0, acc[0][cq][0] + acc[0][cq][1] + acc[0][cq][2], part[cq]);
            if (lv[1]) part[cq] = fmaf(w1, acc[1][cq][0] + acc[1][cq][1] + acc[1][cq][2], part[cq]);
        }
        if (lane < 16) {
            sm.b.red[wave][lane] = part[0];
            sm.b.red[wave][16 + lane] = part[1];
        }
        lds_barrier();
        if (threadIdx.x < 32) {
            const int c = c0c + threadIdx.x;
            const float y = sm.b.red[0][threadIdx.x] + sm.b.red[1][threadIdx.x] + sm.b.red[2][threadIdx.x] +
                            sm.b.red[3][threadIdx.x];
            // runtime/model_runner_v2.py:208: x = x + moe.bfloat16() in bf16
            const float yb = mx::bf16_to_f32(mx::f32_to_bf16_rne(y));
            const uint16_t xn = mx::f32_to_bf16_rne(xown + yb);
            xown = mx::bf16_to_f32(xn);
            wait_stores();   // the previous layer's empty-stores are visible before this publish
            if (l + 1 < L)
                __hip_atomic_store(xbuf + b * a.xwords + c, (uint32_t)xn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                a.x_out[c] = xn;
            // empty these columns in the previous layer's buffer (written again
            // two layers on; its readers, the gate/up workgroups of this layer,
            // are done: h_l is complete)
            __hip_atomic_store(xbuf + bprev * a.xwords + c, kEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.x_all) a.x_all[(int64_t)l * H + c] = xn;
            if (a.y_all) a.y_all[(int64_t)l * H + c] = y;
        }
        if (!STRICT && l + 1 < L) load_w(l + 1);   // streams under the next gate/up phase, after the publish
    }
    if (!live) set_error(a);
    if (threadIdx.x == 0) *memo = c0 + L;
}

__global__ void reset_stack_kernel(uint32_t* ws, int cfg, int words) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < kBufOff / 4) ws[i] = (i == kCfgOff / 4) ? (uint32_t)cfg : 0u;
    if (i < words) ws[kBufOff / 4 + i] = kEmpty;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
int h_words(int E, int Mi) { return (int)(align256((size_t)E * (Mi / 32) * kRecWords * 4) / 4); }
int x_words(int H) { return (int)(align256((size_t)H * 4) / 4); }

}  // namespace

extern "C" size_t mxfp4_decode_stack_workspace_size(int E, int H, int Mi) {
    if (E <= 0 || H <= 0 || Mi <= 0) return 0;
    return kBufOff + (size_t)kNBuf * (h_words(E, Mi) + x_words(H)) * 4;
}

extern "C" int mxfp4_decode_stack_reset(void* workspace, int E, int H, int Mi, void* stream) {
    MXH_REQUIRE(workspace, "decode_stack_reset: null workspace");
    MXH_REQUIRE(E >= 1 && E <= kMaxE && Mi >= 32 && Mi <= 1024 && Mi % 32 == 0 && H >= 512 && H <= 2048 && H % 512 == 0,
                "decode_stack_reset: E=%d H=%d Mi=%d out of range", E, H, Mi);
    const int words = kNBuf * (h_words(E, Mi) + x_words(H));
    const int n = words > kBufOff / 4 ? words : kBufOff / 4;
    hipLaunchKernelGGL(reset_stack_kernel, dim3((n + 255) / 256), dim3(256), 0, mxh::as_stream(stream),
                       static_cast<uint32_t*>(workspace), stack_cfg(E, H, Mi), words);
    return mxh::launch_status("decode_stack_reset");
}

extern "C" int mxfp4_decode_stack_status(const void* workspace, int* error_flag) {
    MXH_REQUIRE(workspace && error_flag, "decode_stack_status: null pointer");
    int host = 0;
    hipError_t e = hipMemcpy(&host, static_cast<const uint8_t*>(workspace) + kErrOff, sizeof host,
                             hipMemcpyDeviceToHost);
    MXH_REQUIRE(e == hipSuccess, "decode_stack_status: %s", hipGetErrorString(e));
    *error_flag = host;
    return MXFP4_OK;
}

extern "C" int mxfp4_moe_decode_stack(const void* x, const int32_t* ids, const float* w, const void* layer_table,
                                      int n_layers, int n_experts, int E, int H, int Mi, void* x_out, void* x_all,
                                      float* y_all, int strict, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    MXH_REQUIRE(x && ids && w && layer_table && x_out && workspace, "moe_decode_stack: null pointer");
    MXH_REQUIRE(n_layers >= 1 && n_layers <= (1 << 16), "moe_decode_stack: n_layers=%d", n_layers);
    MXH_REQUIRE(E >= 1 && E <= kMaxE, "moe_decode_stack: E=%d must be in [1, 8]", E);
    MXH_REQUIRE(n_experts >= E, "moe_decode_stack: n_experts=%d < E=%d", n_experts, E);
    MXH_REQUIRE(H % 512 == 0 && H >= 512 && H <= 2048, "moe_decode_stack: H=%d must be a multiple of 512 in [512, 2048]", H);
    MXH_REQUIRE(Mi % 32 == 0 && Mi >= 32 && Mi <= 1024, "moe_decode_stack: Mi=%d must be a multiple of 32 in [32, 1024]", Mi);
    MXH_REQUIRE(workspace_bytes >= mxfp4_decode_stack_workspace_size(E, H, Mi), "moe_decode_stack: workspace too small");
    MXH_REQUIRE(((uintptr_t)workspace & 255) == 0, "moe_decode_stack: workspace must be 256-byte aligned");
    MXH_REQUIRE(((uintptr_t)x & 15) == 0, "moe_decode_stack: x must be 16-byte aligned");
    const int nA = E * (Mi / 32), nB = H / 32;
    int dev = 0, n_cu = 0;
    MXH_REQUIRE(hipGetDevice(&dev) == hipSuccess &&
                    hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess,
                "moe_decode_stack: cannot query the CU count");
    MXH_REQUIRE(nA + nB <= n_cu && nA + nB <= kMaxWg,
                "moe_decode_stack: E*Mi/32 + H/32 = %d workgroups, more than the %d CUs (one resident workgroup per CU)",
                nA + nB, n_cu);
    const int steps = (Mi / 32 + 3) / 4;
    const void* kern = steps <= 6 ? (strict ? reinterpret_cast<const void*>(&decode_stack_kernel<true, 6>)
                                            : reinterpret_cast<const void*>(&decode_stack_kernel<false, 6>))
                                  : (strict ? reinterpret_cast<const void*>(&decode_stack_kernel<true, 8>)
                                            : reinterpret_cast<const void*>(&decode_stack_kernel<false, 8>));
    int per_cu = 0;
    MXH_REQUIRE(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0) == hipSuccess,
                "moe_decode_stack: occupancy query failed");
    // every workgroup waits on others, so the whole grid must be resident at once
    MXH_REQUIRE((int64_t)per_cu * n_cu >= nA + nB,
                "moe_decode_stack: %d workgroups but only %d x %d can be resident at once", nA + nB, per_cu, n_cu);
    StackArgs a{};
    a.layers = static_cast<const StackLayer*>(layer_table);
    a.ids = ids;
    a.w = w;
    a.x0 = static_cast<const uint16_t*>(x);
    a.x_out = static_cast<uint16_t*>(x_out);
    a.x_all = static_cast<uint16_t*>(x_all);
    a.y_all = y_all;
    a.wp_stride_gu = (int64_t)Mi * (H / 2);
    a.ws_stride_gu = (int64_t)Mi * (H / 32);
    a.wp_stride_dn = (int64_t)H * (Mi / 2);
    a.ws_stride_dn = (int64_t)H * (Mi / 32);
    a.n_layers = n_layers;
    a.n_experts = n_experts;
    a.E = E;
    a.H = H;
    a.Mi = Mi;
    a.cfg = stack_cfg(E, H, Mi);
    a.hwords = h_words(E, Mi);
    a.xwords = x_words(H);
    a.ws = static_cast<uint8_t*>(workspace);
    hipStream_t st = mxh::as_stream(stream);
    const dim3 grid(nA + nB), block(256);
    if (steps <= 6) {
        if (strict) hipLaunchKernelGGL((decode_stack_kernel<true, 6>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((decode_stack_kernel<false, 6>), grid, block, 0, st, a);
    } else {
        if (strict) hipLaunchKernelGGL((decode_stack_kernel<true, 8>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((decode_stack_kernel<false, 8>), grid, block, 0, st, a);
    }
    return mxh::launch_status("moe_decode_stack");
}
