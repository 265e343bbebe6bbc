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
//                           publishes it (three E4M3 terms per value).
//   workgroups [nA, nA+nB)  down + combine: 16 output columns for all E slots.
//                           They load their down weights first, then wait for
//                           all of h (bounded), stage it in LDS, run 2 slots per
//                           wave and combine sum_e w_e*y_e in-workgroup, adding
//                           the bf16 residual as the reference does.
//
// Synchronisation.  Workgroups are dispatched in index order, so every
// gate/up workgroup is resident or finished before any down workgroup waits:
// the wait cannot deadlock.  It is still bounded (kSpinLimit polls); on expiry
// the kernel sets an error flag, skips its work and exits normally.
//   * h travels as 32-bit words, one per value: bytes 0..2 hold the value's
//     three E4M3 terms, and byte 3 of words 0..2 of a (slot, 32-block) record
//     holds the E8M0 code of term 0..2.  A word is its own flag: between uses
//     it holds kEmpty, whose byte 0 is the E4M3 NaN code: term 0 of a finite
//     h never takes it, and a non-finite h makes term 1 a NaN code as well
//     (kEmpty's byte 1 is not), so no published word equals kEmpty.
//     Producers store with agent-scope
//     atomic stores (write-through to the device coherence point).  A
//     consumer first polls one word per wave with agent-scope atomic loads
//     (one request per wave and round while the weights stream: polling a
//     word per thread cost the step ~0.5 us per layer), then reloads all of its
//     words with 16-byte buffer loads carrying the same agent-scope cache
//     policy until none is empty.  (A release/acquire fence pair would
//     instead write back and invalidate a whole L2 per workgroup.)
//   * Every consumer reads every word, so no consumer can empty them; instead
//     there are two buffers, used by alternate launches.  Each workgroup
//     keeps its own launch count ("memo") in the workspace, reads it at start
//     and stores count+1 at the end, so all workgroups agree on the parity.
//     A producer writes its record into buffer (count & 1) and empties its
//     record in the other buffer, which no workgroup of this launch reads
//     and the next launch will use.  No reset is needed between launches or
//     graph replays.  All launches on a workspace must use the same (E, H,
//     Mi): the workspace header records them (mxfp4_decode_layer_reset) and
//     a mismatching launch sets the error flag instead of waiting.
//
// Registers stay at or below 256 VGPRs per lane (184 at Mi <= 768; h is
// staged through LDS, the down K-step count is a template bound), so two
// 256-thread workgroups fit per CU: 512 slots for the E*Mi/32 + H/16 = 320
// workgroups of a layer, every one resident from the start and all weight
// loads in flight at once.  The
// MFMA loops read their operands with clamped, unconditional LDS loads so the
// reads of a phase issue back to back ahead of the MFMA chain.
//
// Activations on the MFMA: there is no bf16 x FP4 MFMA, so the bf16 x (and the
// fp32 h) is split into three E4M3 terms hi + mid + lo with E8M0 32-block
// scales s0, s0 / 16 and s0 / 512 (decode_common.h), that sum back to the
// value to within 2^-13.8 of its block's amax (exactly, for a bf16 x not far
// below its block's amax).  The three terms are rows 0..2 of the 16-row A
// operand of v_mfma_scale_f32_16x16x128_f8f6f4 (A = E4M3, B = E2M1), so one
// MFMA yields all three partial products and y = D[0] + D[1] + D[2]; the other
// 13 rows are zero and cost nothing in an HBM-bound kernel.
#include "attn_merge.h"
#include "attn_partial.h"
#include "decode_common.h"
#include "mx_host.h"

namespace {

using namespace dl;

// workspace layout (bytes)
constexpr int kCfgOff = 0;            // int32 config word written by reset
constexpr int kErrOff = 256;          // int32 error flag
constexpr int kMemoAOff = 1024;       // int32 launch count of gate/up workgroup (s, jb): [8][32]
constexpr int kMemoBOff = 2048;       // int32 launch count of down workgroup cb: [128]
constexpr int kMemoROff = 2560;       // int32 launch count of router workgroup r (fused router): [128]
constexpr int kMemoQOff = 3072;       // int32 launch count of q|k|v workgroup q (fused router tail): [128]
constexpr int kMemoMOff = 6144;       // int32 launch count of attention-merge workgroup h (front): [64]
constexpr int kMemoOOff = 6400;       // int32 launch count of o_proj workgroup o (front): [128]
constexpr int kMemoTOff = 8192;       // int32 launch count of attention chunk workgroup t (next layer): [512]
constexpr int kLogOff = 16384;        // fused router: 8 copies (one per XCD) of (logit, tag) 64-bit words,
                                      // kLogCopy words apart, n_experts <= 256
constexpr int kLogCopy = 256;
constexpr int kHOff = 32768;          // two h buffers of (E, Mi/32, kRecWords) uint32, bufwords apart,
                                      // then (out[c], tag) 64-bit words, c < H, for the q|k|v tail,
                                      // then the front's words: kAttnWords per head of the attention
                                      // output, and (o_proj[c], tag), c < H; then (q|k|v[r], tag)
                                      // for the next layer's attention, r < 8192
constexpr int kMaxRouterWg = 128;     // fused router: 16 logits per workgroup, all logits once per XCD
constexpr int kMaxQkvWg = 128;        // q|k|v tail: 64 rows per workgroup, up to 8192 rows
constexpr int kMaxH = 2048;
constexpr int kMaxHq = 32;            // front: query heads (o_proj K = 4096)
constexpr int kMaxOWg = 128;          // front: o_proj workgroups, 16 rows each
constexpr int kAttnWords = 17;        // front: per head, 16 words of 4 MXFP4 bytes + 1 of the 4 scale codes
constexpr int kMaxAttnWg = 512;       // next layer's attention: chunks x kv heads (max_pos 8192 at 4 kv heads)
constexpr int kWordsAfterH = 2 * kMaxH + kMaxHq * kAttnWords + 64 * kMaxQkvWg;   // 64-bit words after h

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
    const float* logits;      // (n_experts) fp32 router logits: routing computed in-kernel
    // fused router (ROUTE_FUSED): the post-attention residual, RMSNorm and the
    // router projection run inside the launch
    const uint16_t* xres;     // (H) bf16 residual stream
    const float* oproj;       // (H) fp32 added to it as bf16
    const uint16_t* nw;       // (H) bf16 norm weight
    float eps;
    const uint8_t* rwp;       // (n_experts, H/2) + (n_experts, H/32) MXFP4 router weight
    const uint8_t* rws;
    uint16_t* x_out;          // optional (H) bf16(xres + bf16(oproj))
    uint16_t* y_out;          // optional (H) the normed row (the MoE input)
    float* logits_out;        // optional (n_experts) the router logits
    int nr;                   // router workgroups (n_experts / 16)
    // q|k|v tail (ROUTE_FUSED with nq > 0): the next layer's input RMSNorm
    // and q|k|v projection of x_next = bf16(x_out + bf16(out)), in the same
    // launch after the MoE
    const uint16_t* qnw;      // (H) bf16 next layer's input norm weight
    const uint8_t* qwp;       // (Nq, H/2) + (Nq, H/32) MXFP4 q|k|v weight
    const uint8_t* qws;
    float* qkv_out;           // (Nq) fp32
    uint16_t* xn_out;         // optional (H) bf16 x_next
    int nq, Nq;               // tail workgroups (ceil(Nq / 64)) and rows
    // attention merge + o_proj front (ROUTE_FUSED with nm > 0): the launch
    // first merges the token's decode-attention chunk records (one workgroup
    // per query head) and runs o_proj on the MXFP4 of the result; the o_proj
    // output then reaches the other workgroups as (value, tag) words instead
    // of through `oproj`
    const float* apart;       // attention chunk records of the token: head h at + h*nchunk*kPart
    const int32_t* dpos;      // the token's position
    int nchunk, max_pos;
    uint8_t* aq_out;          // optional (Hq*128/2) + (Hq*128/32) MXFP4 attention output
    uint8_t* as_out;
    const uint8_t* owp;       // (H, 2048) + (H, 128) MXFP4 o_proj weight (K = 4096)
    const uint8_t* ows;
    float* oproj_out;         // optional (H) fp32 o_proj output
    int nm, no;               // merge workgroups (Hq = 32) and o_proj workgroups (H / 16)
    // the next layer's attention chunk pass (with the q|k|v tail, nat > 0):
    // nat = nchunk * Hkv workgroups after the tail take q and the new k / v
    // rows from the tail's (value, tag) words and write the next layer's KV
    // rows and chunk records (apart_n), which the next launch merges
    float* apart_n;
    uint8_t* kvk_n;
    uint8_t* kvv_n;
    const uint16_t* qn_n;     // next layer's q / k head RMSNorm weights (128) bf16
    const uint16_t* kn_n;
    float theta;
    int codec;
    int nat, hkv;
    int n_experts;            // experts per layer (logits routing)
    int norm;                 // renormalise the top-E weights (logits routing)
    int32_t* ids_out;         // optional (E) ids / weights written by workgroup 0 (logits routing)
    float* w_out;
    int E, H, Mi;
    int cfg;                  // expected workspace config word
    int bufwords;             // uint32 words between the two h buffers
    float* out;               // (H) fp32 moe output
    uint16_t* resid;          // (H) bf16 x + bf16(out), or null
    uint8_t* ws;              // workspace base
};

__host__ __device__ constexpr int layer_cfg(int E, int H, int Mi) {
    return 0x5A000000 | (E << 16) | ((H / 512) << 12) | (Mi / 32);
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

__device__ __forceinline__ void set_error(const LayerArgs& a) {
    __hip_atomic_store(reinterpret_cast<int*>(a.ws + kErrOff), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

union Smem {
    struct {                                       // gate/up workgroups
        uint4 zero[2];                             // operand source of the zero rows / steps
        uint8_t x8[kTerms][2048];                  // E4M3 terms of x (H <= 2048)
        uint8_t xsc[kTerms][64];
        float red[4][4][16];
        float h[2][32];
    } a;
    struct {                                       // down workgroups
        uint4 zero[2];                             // operand source of the zero rows / blocks
        uint32_t code127[4];                       // [0]: scale source of the zero rows / blocks (h8 stays 16-B aligned)
        uint8_t h8[kMaxE * kTerms * 1024];         // E4M3 terms of h, [record][term][32], record = slot*Mi/32 + block
        uint32_t hsc[kMaxE * 32];                  // [record]: codes of terms 0..2
        float red[4][16];
        int abort;
    } b;
    struct {                                       // router workgroups (fused router)
        uint4 zero[2];
        uint8_t xq[1024];                          // the normed row's MXFP4 (H <= 2048)
        uint8_t xs[64];
        float red[4][16];
    } r;
    am::MergeLds m;                                // attention-merge workgroups (front)
    ap::AttnLds<1, true> t;                        // next layer's attention chunk workgroups
    struct {                                       // o_proj workgroups (front)
        uint8_t aq[kMaxHq * 64];                   // the attention output's MXFP4 (K = 4096)
        uint8_t as[kMaxHq * 4];
        float red[8][16];                          // row sums of the eight K parts
    } o;
};

// The (out[c], tag) words the down workgroups publish for the q|k|v tail.
__device__ __forceinline__ uint64_t* out_words(const LayerArgs& a) {
    return reinterpret_cast<uint64_t*>(a.ws + kHOff + (size_t)2 * a.bufwords * 4);
}
// The front's words: the attention output (kAttnWords per head), then o_proj's.
__device__ __forceinline__ uint64_t* attn_words(const LayerArgs& a) { return out_words(a) + kMaxH; }
__device__ __forceinline__ uint64_t* oproj_words(const LayerArgs& a) {
    return attn_words(a) + kMaxHq * kAttnWords;
}
__device__ __forceinline__ uint64_t* qkv_words(const LayerArgs& a) { return oproj_words(a) + kMaxH; }

// Word position of element e among the o_proj words and the MoE output words
// (H = 2048, thread t of 256 reading elements 8t .. 8t+7): element 8t + i sits
// at 512 (i >> 1) + 2t + (i & 1), so a thread's elements are four adjacent word
// pairs and each of its four 16-byte loads is lane-contiguous (8 cache lines a
// load instead of 32 for eight 8-byte loads at a 64-byte lane stride).
__device__ __forceinline__ int opos(int e) { return ((e & 6) << 8) | ((e >> 3) << 1) | (e & 1); }

// o_proj output elements 8t .. 8t+7 of thread t: from `oproj`, or with the
// front from this launch's o_proj words -- one probe word per wave (the first
// column of the wave's last thread), then the thread's words until all carry
// `tag`.  Returns false when the bounded wait expired (values then zero).
__device__ __forceinline__ bool load_oproj(const LayerArgs& a, uint32_t tag, float (&of)[8]) {
    const int k0 = 8 * (int)threadIdx.x, wave = threadIdx.x >> 6;
    if (a.nm == 0) {
        const float4 o0 = *reinterpret_cast<const float4*>(a.oproj + k0);
        const float4 o1 = *reinterpret_cast<const float4*>(a.oproj + k0 + 4);
        of[0] = o0.x; of[1] = o0.y; of[2] = o0.z; of[3] = o0.w;
        of[4] = o1.x; of[5] = o1.y; of[6] = o1.z; of[7] = o1.w;
        return true;
    }
    const uint64_t* words = oproj_words(a);
    int spins = 0;
    bool ok = true;
    while (true) {
        const uint64_t w0 = __hip_atomic_load(words + opos(8 * (64 * wave + 63)), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane((uint32_t)(w0 >> 32)) == tag) break;
        if (++spins >= kSpinLimit) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    // agent-scope (sc1) 16-byte loads of two (value, tag) words each
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(words), (short)0, kMaxH * 8, 0x00020000);
    while (ok) {
        bool pending = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const v4u w = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)((opos(k0 + 2 * j)) * 8), 0, 16);
            of[2 * j] = __uint_as_float(w.x);
            of[2 * j + 1] = __uint_as_float(w.z);
            pending |= w.y != tag || w.w != tag;
        }
        if (!pending) break;
        if (++spins >= kSpinLimit) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
        asm volatile("" ::: "memory");
    }
    if (!ok) {
#pragma unroll
        for (int i = 0; i < 8; ++i) of[i] = 0.0f;
    }
    return ok;
}

// The post-attention residual and RMSNorm of one row for the fused router,
// thread t holding elements 8t .. 8t+7 (H = 2048, 256 threads): v = bf16(x +
// bf16(o)), y = bf16(bf16(v * rstd) * w) -- the arithmetic of
// mxfp4_rmsnorm_quant / mxfp4_rmsnorm_lin_pq (runtime/model_runner.py:20-25),
// including its order of the sum of squares, so y equals theirs bit for bit.
// q, wq4: the thread's residual and norm weight elements (NormIn, loaded
// before the o_proj wait); of: its o_proj elements (load_oproj).  Every
// thread of the workgroup must call it (one barrier).
struct NormIn {
    uint4 q, wq4;
    __device__ __forceinline__ explicit NormIn(const LayerArgs& a)
        : q(*reinterpret_cast<const uint4*>(a.xres + 8 * threadIdx.x)),
          wq4(*reinterpret_cast<const uint4*>(a.nw + 8 * threadIdx.x)) {}
};
__device__ __forceinline__ void fused_norm_row(const LayerArgs& a, float* nred, const NormIn& in, const float (&of)[8],
                                               float (&v)[8], float (&y)[8]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint4 q = in.q, wq4 = in.wq4;
    const uint32_t xw[4] = {q.x, q.y, q.z, q.w};
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float xi = mx::bf16_to_f32((uint16_t)(xw[i / 2] >> (16 * (i & 1))));
        v[i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(xi + mx::bf16_to_f32(mx::f32_to_bf16_rne(of[i]))));
        ss = fmaf(v[i], v[i], ss);
    }
    ss = mx::wave_sum_butterfly(ss);   // the xor-32..1 butterfly of rmsnorm_lin_pq
    if (lane == 0) nred[wave] = ss;
    __syncthreads();
    const float var = ((nred[0] + nred[1]) + (nred[2] + nred[3])) / (float)2048;
    const float rr = 1.0f / sqrtf(var + a.eps);
    const uint32_t ww[4] = {wq4.x, wq4.y, wq4.z, wq4.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float wi = mx::bf16_to_f32((uint16_t)(ww[i / 2] >> (16 * (i & 1))));
        const float t = mx::bf16_to_f32(mx::f32_to_bf16_rne(v[i] * rr));
        y[i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(t * wi));
    }
}

// The router logits of this launch from the workspace: element i*64 + lane
// into lv[i], waiting (bounded) until every word carries this launch's tag.
// The copy read is the one the router workgroups of this workgroup's XCD
// write (blockIdx.x % 8: workgroups are dealt to the 8 XCDs round-robin), so
// the hand-off stays in one L2; any copy holds every logit.
template <int NPL>
__device__ __forceinline__ bool poll_logits(const LayerArgs& a, uint32_t tag, float (&lv)[NPL]) {
    const uint64_t* words = reinterpret_cast<const uint64_t*>(a.ws + kLogOff) + (blockIdx.x & 7) * kLogCopy;
    const int lane = threadIdx.x & 63;
    int spins = 0;
    // the last logit first, one request per wave and round
    while (true) {
        const uint64_t w = __hip_atomic_load(words + (a.n_experts - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane((uint32_t)(w >> 32)) == tag) break;
        if (++spins >= kSpinLimit) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    while (true) {
        bool pending = false;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int idx = i * 64 + lane;
            lv[i] = 0.0f;
            if (idx < a.n_experts) {
                const uint64_t w = __hip_atomic_load(words + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                lv[i] = __uint_as_float((uint32_t)w);
                pending |= (uint32_t)(w >> 32) != tag;
            }
        }
        if (__builtin_amdgcn_ballot_w64(pending) == 0) return true;
        if (++spins >= kSpinLimit) return false;
        __builtin_amdgcn_s_sleep(2);
        asm volatile("" ::: "memory");
    }
}

// Router workgroup ri (fused router): logits [16c, 16c + 16), c = ri / 8, of
// the normed row -- its MXFP4 (the reference quantizes the bf16 row,
// prequant) times the router's MXFP4 rows on v_mfma_scale_f32_16x16x128_f8f6f4
// (row 0 of A is the row, rows 1..15 zero), K split over the four waves,
// partial sums added in wave order -- published as (value, tag) words into
// the logit copy of its XCD (blockIdx.x % 8), read by that XCD's gate/up and
// down workgroups: every XCD computes all logits (8 x 16 router rows of
// 1 KB each), so the hand-off to the routing stays in one L2.  The words are
// workgroup-scope stores (they stay in this XCD's L2, where the readers'
// agent-scope polls find them): that relies on the round-robin dispatch of
// workgroups to XCDs, which the copy index assumes; under another placement
// a reader sees only an older tag, its bounded wait expires and the error
// flag is set -- it never takes a stale logit.  Router workgroup 0 also
// writes x_out / y_out.
__device__ __forceinline__ void router_wg(const LayerArgs& a, Smem& sm, float* nred, int ri) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int chunk = ri >> 3;
    int* memo = reinterpret_cast<int*>(a.ws + kMemoROff) + ri;
    const int launch = *memo;
    const int cfg = *reinterpret_cast<const int*>(a.ws + kCfgOff);
    // weights first: row 16c + r, blocks 16*wave + 4g .. +3 (64 contiguous bytes) and their scales
    const int blk0 = 16 * wave + 4 * g;
    const int row = min(16 * chunk + r, a.n_experts - 1);
    const uint8_t* wr = a.rwp + (int64_t)row * 1024 + blk0 * 16;
    uint4 wq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wq[i] = *reinterpret_cast<const uint4*>(wr + 16 * i);
    const uint32_t wsc = *reinterpret_cast<const uint32_t*>(a.rws + (int64_t)row * 64 + blk0);
    const NormIn nin(a);
    float of[8], v[8], y[8];
    if (!load_oproj(a, (uint32_t)(launch + 1), of)) set_error(a);
    fused_norm_row(a, nred, nin, of, v, y);
    // MXFP4 of y (bf16-exact values): block tid / 4, the block's four threads
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, __builtin_fabsf(y[i]));
    am = fmaxf(am, mx::dpp<mx::kDppQuadXor1>(am));
    am = fmaxf(am, mx::dpp<mx::kDppQuadXor2>(am));
    const uint32_t code = mx::e8m0_code(am);
    *reinterpret_cast<uint32_t*>(sm.r.xq + 4 * tid) = mx::e2m1_pack8_short(y, mx::e8m0_inv_scale(code));
    if ((tid & 3) == 0) sm.r.xs[tid >> 2] = (uint8_t)code;
    if (tid < 2) sm.r.zero[tid] = make_uint4(0, 0, 0, 0);
    if (ri == 0) {
        const int k0 = 8 * tid;
        uint32_t xo[4], yo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xo[i] = (uint32_t)mx::f32_to_bf16_rne(v[2 * i]) | ((uint32_t)mx::f32_to_bf16_rne(v[2 * i + 1]) << 16);
            yo[i] = (uint32_t)mx::f32_to_bf16_rne(y[2 * i]) | ((uint32_t)mx::f32_to_bf16_rne(y[2 * i + 1]) << 16);
        }
        if (a.x_out) *reinterpret_cast<uint4*>(a.x_out + k0) = make_uint4(xo[0], xo[1], xo[2], xo[3]);
        if (a.y_out) *reinterpret_cast<uint4*>(a.y_out + k0) = make_uint4(yo[0], yo[1], yo[2], yo[3]);
    }
    __syncthreads();
    mx::v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4* pa = r == 0 ? reinterpret_cast<const uint4*>(sm.r.xq + (blk0 + i) * 16) : &sm.r.zero[0];
        const uint32_t asc = r == 0 ? (uint32_t)sm.r.xs[blk0 + i] : 127u;
        acc = mx::mfma16_fp4(*pa, wq[i], acc, asc, (wsc >> (8 * i)) & 0xFFu);
    }
    mx::pin(acc);
    // D[0][lane] (lane < 16): the wave's K quarter of logit 16ri + lane
    if (lane < 16) sm.r.red[wave][lane] = acc[0];
    __syncthreads();
    if (tid < 16) {
        const float lg = (sm.r.red[0][tid] + sm.r.red[1][tid]) + (sm.r.red[2][tid] + sm.r.red[3][tid]);
        const int idx = 16 * chunk + tid;
        if (idx < a.n_experts) {
            uint64_t* words = reinterpret_cast<uint64_t*>(a.ws + kLogOff) + (blockIdx.x & 7) * kLogCopy;
            __hip_atomic_store(words + idx, (uint64_t)__float_as_uint(lg) | ((uint64_t)(uint32_t)(launch + 1) << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (a.logits_out && (ri & 7) == 0) a.logits_out[idx] = lg;
        }
    }
    if (tid == 0) {
        // (the launch counts of the router slots this launch has no
        // workgroup for move on with gate/up workgroup 0)
        *memo = launch + 1;
        if (cfg != a.cfg) set_error(a);
    }
}

// Attention-merge workgroup h (front): merges head h's chunk records of the
// token with attn_final_kernel's arithmetic (am::merge_head) and publishes
// the MXFP4 of bf16(o) as kAttnWords (value, tag) words: word j < 16 holds
// the packed bytes 4j .. 4j+3 of the head's 64, word 16 its four block
// codes.  A position outside [0, max_pos) publishes zeros (attn_final_kernel
// writes nothing there).
__device__ __forceinline__ void merge_wg(const LayerArgs& a, Smem& sm, int h) {
    const int lane = threadIdx.x & 63;
    int* memo = reinterpret_cast<int*>(a.ws + kMemoMOff) + h;
    const int launch = *memo;
    const int cfg = *reinterpret_cast<const int*>(a.ws + kCfgOff);
    const int pos = *a.dpos;
    uint32_t bytes = 0, code = 127;
    if (pos >= 0 && pos < a.max_pos) {
        float r0, r1;
        if (!am::merge_head(a.apart + (int64_t)h * a.nchunk * am::kPart, pos / am::kChunk + 1, sm.m, r0, r1))
            return;   // waves 1..3
        am::quant_head_row(r0, r1, bytes, code);
    } else if (threadIdx.x >= 64) {
        return;
    }
    const uint64_t tag = (uint64_t)(uint32_t)(launch + 1) << 32;
    uint64_t* w = attn_words(a) + h * kAttnWords;
    const bool cfg_ok = cfg == a.cfg;
    const uint32_t codes = (uint32_t)__builtin_amdgcn_readlane((int)code, 0) |
                           ((uint32_t)__builtin_amdgcn_readlane((int)code, 16) << 8) |
                           ((uint32_t)__builtin_amdgcn_readlane((int)code, 32) << 16) |
                           ((uint32_t)__builtin_amdgcn_readlane((int)code, 48) << 24);
    if (cfg_ok) {
        if ((lane & 3) == 0) __hip_atomic_store(w + (lane >> 2), (uint64_t)bytes | tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) __hip_atomic_store(w + 16, (uint64_t)codes | tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (a.aq_out) {
        if ((lane & 3) == 0) *reinterpret_cast<uint32_t*>(a.aq_out + h * 64 + lane) = bytes;
        if ((lane & 15) == 0) a.as_out[h * 4 + lane / 16] = (uint8_t)code;
    }
    if (lane == 0) {
        *memo = launch + 1;
        if (!cfg_ok) set_error(a);
    }
}

// o_proj workgroup oi (front): rows 16oi .. 16oi+15 of o_proj (K = 4096) on
// this launch's attention output, with the arithmetic mxfp4_lin_pq uses for
// one row at this shape (lin_small_kernel<1, 8>): K in eight parts of four
// MFMA steps (block 16p + 4s + g at step s of part p), two parts per wave
// here, the part sums added in part order -- so the rows equal lin_pq's bit
// for bit.  Published as (value, tag) words, and written to oproj_out.
__device__ __forceinline__ void oproj_wg(const LayerArgs& a, Smem& sm, int oi) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    int* memo = reinterpret_cast<int*>(a.ws + kMemoOOff) + oi;
    const int launch = *memo;
    const int cfg = *reinterpret_cast<const int*>(a.ws + kCfgOff);
    constexpr int kRowB = kMaxHq * 64, kRowS = kMaxHq * 4;   // bytes and scale bytes of a weight row
    const int row = 16 * oi + r;
    const uint8_t* wr = a.owp + (int64_t)row * kRowB + g * 16;
    uint4 wq[2][4], sc4[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int p = 2 * wave + q;
#pragma unroll
        for (int s = 0; s < 4; ++s) wq[q][s] = *reinterpret_cast<const uint4*>(wr + (16 * p + 4 * s) * 16);
        sc4[q] = *reinterpret_cast<const uint4*>(a.ows + (int64_t)row * kRowS + 16 * p);
    }
    // the attention output words: thread t takes words t, t + 256, t + 512;
    // first one probe word per wave (head 31's codes, published last)
    const uint64_t* words = attn_words(a);
    constexpr int kW = kMaxHq * kAttnWords;
    const uint32_t tag = (uint32_t)(launch + 1);
    bool ok = cfg == a.cfg;
    int spins = 0;
    while (ok) {
        const uint64_t w0 = __hip_atomic_load(words + kW - 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane((uint32_t)(w0 >> 32)) == tag) break;
        if (++spins >= kSpinLimit) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    uint64_t wv[3];
    while (ok) {
        bool pending = false;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int idx = min(tid + 256 * i, kW - 1);
            wv[i] = __hip_atomic_load(words + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            pending |= (uint32_t)(wv[i] >> 32) != tag;
        }
        if (!pending) break;
        if (++spins >= kSpinLimit) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
        asm volatile("" ::: "memory");
    }
    if (__syncthreads_or(!ok)) {
        if (tid == 0) {
            set_error(a);
            *memo = launch + 1;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int idx = tid + 256 * i;
        if (idx < kW) {
            const int h = idx / kAttnWords, j = idx - h * kAttnWords;
            uint8_t* dst = j < 16 ? sm.o.aq + h * 64 + 4 * j : sm.o.as + h * 4;
            *reinterpret_cast<uint32_t*>(dst) = (uint32_t)wv[i];
        }
    }
    __syncthreads();
    mx::v4f acc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int p = 2 * wave + q;
        acc[q] = (mx::v4f){0.f, 0.f, 0.f, 0.f};
        const uint32_t sw[4] = {sc4[q].x, sc4[q].y, sc4[q].z, sc4[q].w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int c = 16 * p + 4 * s + g;
            const uint4 aq = *reinterpret_cast<const uint4*>(sm.o.aq + c * 16);
            acc[q] = mx::mfma16_fp4(aq, wq[q][s], acc[q], (uint32_t)sm.o.as[c], (sw[s] >> (8 * g)) & 0xFFu);
        }
    }
    mx::pin(acc[0]);   // the whole MFMA chain before the lane < 16 branch
    mx::pin(acc[1]);
    if (lane < 16) {
        sm.o.red[2 * wave][lane] = acc[0][0];
        sm.o.red[2 * wave + 1][lane] = acc[1][0];
    }
    __syncthreads();
    if (tid < 16) {
        float t = sm.o.red[0][tid];
#pragma unroll
        for (int p = 1; p < 8; ++p) t += sm.o.red[p][tid];
        __hip_atomic_store(oproj_words(a) + opos(16 * oi + tid), (uint64_t)__float_as_uint(t) | ((uint64_t)tag << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.oproj_out) a.oproj_out[16 * oi + tid] = t;
    }
    if (tid == 0) *memo = launch + 1;
}

// q|k|v values for the next layer's attention chunk pass from the tail's
// (value, tag) words (ap::attn_partial_body's source): one probe word per
// wave, then the rows until every word carries the tag.  Rows repeated in
// the wave's list (clamped rows of absent tokens: at M = 1 the q rows of the
// second token slot and all k / v tasks) are loaded once.  On expiry the
// error flag is set and the values are zero.
struct TaggedQkv {
    static constexpr bool kWaits = true;
    const uint64_t* words;
    uint32_t tag;
    int* err;
    template <int N>
    __device__ __forceinline__ static bool load_rows(const uint64_t* words, uint32_t tag, const int64_t (&o)[N],
                                                     float (&va)[N], float (&vb)[N]) {
        const int lane = threadIdx.x & 63;
        bool pending = false;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int dup = -1;
#pragma unroll
            for (int k = 0; k < i; ++k) dup = (dup < 0 && o[k] == o[i]) ? k : dup;
            if (dup < 0) {
                const uint64_t wa = __hip_atomic_load(words + o[i] + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t wb = __hip_atomic_load(words + o[i] + lane + 64, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
                va[i] = __uint_as_float((uint32_t)wa);
                vb[i] = __uint_as_float((uint32_t)wb);
                pending |= (uint32_t)(wa >> 32) != tag || (uint32_t)(wb >> 32) != tag;
            } else {
                va[i] = va[dup];
                vb[i] = vb[dup];
            }
        }
        return pending;
    }
    template <int QR, int NR>
    __device__ __forceinline__ bool fetch(const int64_t (&qo)[QR], const int64_t (&ko)[NR], float (&qa)[QR],
                                          float (&qb)[QR], float (&ka)[NR], float (&kb)[NR]) const {
        int spins = 0;
        bool ok = true;
        while (true) {
            const uint64_t w = __hip_atomic_load(words + ko[NR - 1] + 127, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__builtin_amdgcn_readfirstlane((uint32_t)(w >> 32)) == tag) break;
            if (++spins >= kSpinLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        while (ok) {
            bool pending = load_rows<QR>(words, tag, qo, qa, qb);
            pending |= load_rows<NR>(words, tag, ko, ka, kb);
            if (__builtin_amdgcn_ballot_w64(pending) == 0) break;
            if (++spins >= kSpinLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            asm volatile("" ::: "memory");
        }
        if (!ok) {
#pragma unroll
            for (int i = 0; i < QR; ++i) qa[i] = qb[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < NR; ++j) ka[j] = kb[j] = 0.0f;
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return ok;
    }
};

// Attention chunk workgroup ti (next layer, after the q|k|v tail): chunk ti
// % nchunk of kv head ti / nchunk, attn_partial_kernel's work for one token
// (ap::attn_partial_body, 8 query heads per kv head) with q and the new k /
// v rows from this launch's q|k|v words.  Its K / V cache loads are issued
// at dispatch, while the MoE runs.
__device__ __forceinline__ void attn_wg(const LayerArgs& a, Smem& sm, int ti) {
    int* memo = reinterpret_cast<int*>(a.ws + kMemoTOff) + ti;
    const int launch = *memo;
    const TaggedQkv src{qkv_words(a), (uint32_t)(launch + 1), reinterpret_cast<int*>(a.ws + kErrOff)};
    const ap::QkvIn fz{nullptr, a.qn_n, a.kn_n, a.eps, a.theta, a.codec, a.kvk_n, a.kvv_n};
    ap::attn_partial_body<8, 1, true>(sm.t, src, ti % a.nchunk, ti / a.nchunk, 0, nullptr, a.kvk_n, a.kvv_n, nullptr,
                                      a.apart_n, a.dpos, 1, 8 * a.hkv, a.hkv, a.max_pos, a.nchunk,
                                      1.0f / sqrtf((float)am::kD), fz);
    if (threadIdx.x == 0) *memo = launch + 1;
}

// q|k|v tail workgroup qi (fused router, nq > 0): rows 64qi .. 64qi+63 of
// the next layer's q|k|v projection, wave w rows 64qi + 16w .. +15.  The
// weights are loaded first and stream while the MoE runs; the workgroup then
// waits (bounded) for this launch's MoE output words of its thread's eight
// columns, forms x_next = bf16(x' + bf16(out)) with x' = bf16(x + bf16(o)) as
// fused_norm_row computes it, and runs mxfp4_rmsnorm_lin_pq's arithmetic:
// the RMSNorm (same order of the sum of squares), the MXFP4 row, and the
// GEMV with K split in four parts of four MFMA steps (block 16p + 4s + g at
// step s of part p), the parts added in order -- so x_next equals a separate
// mxfp4_rmsnorm_lin_pq call's bit for bit, and so does qkv_out where that
// call splits K in four (4081 to 8192 rows: 5120 for 32 + 2 x 4 heads of 128).
__device__ __forceinline__ void qkv_wg(const LayerArgs& a, Smem& sm, float* nred, int qi) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    int* memo = reinterpret_cast<int*>(a.ws + kMemoQOff) + qi;
    const int launch = *memo;
    const int cfg = *reinterpret_cast<const int*>(a.ws + kCfgOff);
    const int row_i = 64 * qi + 16 * wave + r;
    const int row = min(row_i, a.Nq - 1);
    const uint8_t* wr = a.qwp + (int64_t)row * (kMaxH / 2) + g * 16;
    uint4 wq[4][4];
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int s = 0; s < 4; ++s) wq[p][s] = *reinterpret_cast<const uint4*>(wr + (16 * p + 4 * s) * 16);
    uint4 sc4[4];   // the row's 64 scale bytes: block 16p + 4s + g is byte g of dword s of sc4[p]
#pragma unroll
    for (int p = 0; p < 4; ++p) sc4[p] = *reinterpret_cast<const uint4*>(a.qws + (int64_t)row * (kMaxH / 32) + 16 * p);
    const int k0 = 8 * tid;
    const uint4 q = *reinterpret_cast<const uint4*>(a.xres + k0);
    const uint4 wn = *reinterpret_cast<const uint4*>(a.qnw + k0);
    // this launch's MoE output of columns k0 .. k0+7 (out words at opos(column): four
    // lane-contiguous 16-byte loads)
    const __amdgpu_buffer_rsrc_t yrs =
        __builtin_amdgcn_make_buffer_rsrc(out_words(a), (short)0, kMaxH * 8, 0x00020000);
    const uint32_t tag = (uint32_t)(launch + 1);
    float of[8], yo[8];
    // one probe word per wave first (the first column of the wave's last
    // thread; one request per round while the weights stream), then every
    // thread's words until all carry the tag
    bool ok = cfg == a.cfg && load_oproj(a, tag, of);
    int spins = 0;
    while (ok) {
        const uint64_t w0 = __hip_atomic_load(out_words(a) + opos(8 * (64 * wave + 63)), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane((uint32_t)(w0 >> 32)) == tag) break;
        if (++spins >= kSpinLimit) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    while (ok) {
        bool pending = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const v4u w = __builtin_amdgcn_raw_buffer_load_b128(yrs, (uint32_t)(opos(k0 + 2 * j) * 8), 0, 16);
            yo[2 * j] = __uint_as_float(w.x);
            yo[2 * j + 1] = __uint_as_float(w.z);
            pending |= w.y != tag || w.w != tag;
        }
        if (!pending) break;
        if (++spins >= kSpinLimit) {
            ok = false;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
        asm volatile("" ::: "memory");
    }
    if (__syncthreads_or(!ok)) {
        if (tid == 0) {
            set_error(a);
            *memo = launch + 1;
        }
        return;
    }
    const uint32_t xw[4] = {q.x, q.y, q.z, q.w};
    float v[8];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float xi = mx::bf16_to_f32((uint16_t)(xw[i / 2] >> (16 * (i & 1))));
        const float xp = mx::bf16_to_f32(mx::f32_to_bf16_rne(xi + mx::bf16_to_f32(mx::f32_to_bf16_rne(of[i]))));
        v[i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(xp + mx::bf16_to_f32(mx::f32_to_bf16_rne(yo[i]))));
        ss = fmaf(v[i], v[i], ss);
    }
    ss = mx::wave_sum_butterfly(ss);   // the xor-32..1 butterfly of rmsnorm_lin_pq
    if (lane == 0) nred[wave] = ss;
    __syncthreads();
    const float var = ((nred[0] + nred[1]) + (nred[2] + nred[3])) / (float)kMaxH;
    const float rr = 1.0f / sqrtf(var + a.eps);
    const uint32_t ww[4] = {wn.x, wn.y, wn.z, wn.w};
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float wi = mx::bf16_to_f32((uint16_t)(ww[i / 2] >> (16 * (i & 1))));
        const float t = mx::bf16_to_f32(mx::f32_to_bf16_rne(v[i] * rr));
        y[i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(t * wi));
    }
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, __builtin_fabsf(y[i]));
    am = fmaxf(am, mx::dpp<mx::kDppQuadXor1>(am));
    am = fmaxf(am, mx::dpp<mx::kDppQuadXor2>(am));
    const uint32_t code = mx::e8m0_code(am);
    *reinterpret_cast<uint32_t*>(sm.r.xq + 4 * tid) = mx::e2m1_pack8_short(y, mx::e8m0_inv_scale(code));
    if ((tid & 3) == 0) sm.r.xs[tid >> 2] = (uint8_t)code;
    if (qi == 0 && a.xn_out) {
        uint32_t xo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            xo[i] = (uint32_t)mx::f32_to_bf16_rne(v[2 * i]) | ((uint32_t)mx::f32_to_bf16_rne(v[2 * i + 1]) << 16);
        *reinterpret_cast<uint4*>(a.xn_out + k0) = make_uint4(xo[0], xo[1], xo[2], xo[3]);
    }
    __syncthreads();
    // every A row is the normed row (as mxfp4_rmsnorm_lin_pq at M = 1), D[0][r] = row 16w + r
    mx::v4f acc[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        acc[p] = (mx::v4f){0.f, 0.f, 0.f, 0.f};
        const uint32_t sw[4] = {sc4[p].x, sc4[p].y, sc4[p].z, sc4[p].w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int c = 16 * p + 4 * s + g;
            const uint4 aq = *reinterpret_cast<const uint4*>(sm.r.xq + c * 16);
            acc[p] = mx::mfma16_fp4(aq, wq[p][s], acc[p], (uint32_t)sm.r.xs[c], (sw[s] >> (8 * g)) & 0xFFu);
        }
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) mx::pin(acc[p]);   // the whole MFMA chain before the lane < 16 branch
    float t = acc[0][0];
    t += acc[1][0];
    t += acc[2][0];
    t += acc[3][0];
    if (lane < 16 && row_i < a.Nq) {
        a.qkv_out[row_i] = t;
        if (a.nat > 0)   // for the next layer's attention workgroups of this launch
            __hip_atomic_store(qkv_words(a) + row_i, (uint64_t)__float_as_uint(t) | ((uint64_t)tag << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid == 0) {
        *memo = launch + 1;
        if (cfg != a.cfg) set_error(a);
    }
}

// Where the routing comes from: kernel arguments, device arrays, or router
// logits in device memory (softmax / top-E / renormalise computed by every
// wave at entry, mx::wave_topk).
enum { ROUTE_HOST = 0, ROUTE_DEV_IDS = 1, ROUTE_LOGITS = 2, ROUTE_FUSED = 3 };
constexpr int kRouteNpl = 4;          // logits routing: up to 256 experts

template <int ROUTE, int MS>
__global__ __launch_bounds__(256) void decode_layer_kernel(LayerArgs a) {
    __shared__ __align__(16) Smem sm;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int g = lane >> 4;
    const int rr = r < kTerms ? r : 0;     // A-operand term row read by this lane (rows >= 3 are zero)
    const int nblk_mi = a.Mi >> 5;
    const int nA = a.E * nblk_mi;
    constexpr bool kLogitRoute = ROUTE == ROUTE_LOGITS || ROUTE == ROUTE_FUSED;
    // fused router: workgroups [0, nm) merge the attention heads and [nm,
    // nm + no) run o_proj (the front, nm = no = 0 without it), the next nr
    // compute the router logits; the gate/up and down workgroups follow them
    const int nfront = ROUTE == ROUTE_FUSED ? a.nm + a.no : 0;
    const int bid = (int)blockIdx.x - (ROUTE == ROUTE_FUSED ? nfront + a.nr : 0);
    __shared__ float nred[4];
    if constexpr (ROUTE == ROUTE_FUSED) {
        if ((int)blockIdx.x < a.nm) {
            merge_wg(a, sm, (int)blockIdx.x);
            return;
        }
        if ((int)blockIdx.x < nfront) {
            oproj_wg(a, sm, (int)blockIdx.x - a.nm);
            return;
        }
        if (bid < 0) {
            router_wg(a, sm, nred, (int)blockIdx.x - nfront);
            return;
        }
        // q|k|v tail workgroups follow the down workgroups, the next layer's
        // attention chunk workgroups follow them
        if (bid >= nA + (a.H >> 4) + a.nq) {
            attn_wg(a, sm, bid - nA - (a.H >> 4) - a.nq);
            return;
        }
        if (bid >= nA + (a.H >> 4)) {
            qkv_wg(a, sm, nred, bid - nA - (a.H >> 4));
            return;
        }
    }
    uint32_t* hbuf = reinterpret_cast<uint32_t*>(a.ws + kHOff);
    // logits routing: lane r < E of every wave holds rank r (id, weight)
    int rid = 0;
    float rw = 0.0f;
    // gate/up workgroups: x is loaded before the routing, so its latency
    // overlaps the top-k (the weight loads need the routing, x does not);
    // with the fused router, x is the normed row, computed here from the
    // residual inputs while the router workgroups run
    const int k0 = threadIdx.x * 8;
    uint4 xq = make_uint4(0, 0, 0, 0);
    float yf[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // fused router: this launch's tag is the workgroup's own launch count + 1
    const int* memo0 = reinterpret_cast<const int*>(a.ws) +
                       (bid < nA ? kMemoAOff / 4 + (bid % a.E) * 32 + bid / a.E : kMemoBOff / 4 + (bid - nA));
    if constexpr (ROUTE == ROUTE_FUSED) {
        if (bid < nA) {
            const NormIn nin(a);
            float of[8], vf[8];
            if (!load_oproj(a, (uint32_t)(*memo0 + 1), of)) set_error(a);
            fused_norm_row(a, nred, nin, of, vf, yf);
        }
    } else {
        if (bid < nA && k0 < a.H) xq = *reinterpret_cast<const uint4*>(a.x + k0);
    }
    if constexpr (ROUTE == ROUTE_LOGITS) {
        mx::wave_topk<kRouteNpl>(a.logits, a.n_experts, a.E, a.norm, rid, rw);
    }
    if constexpr (ROUTE == ROUTE_FUSED) {
        float lv[kRouteNpl];
        if (!poll_logits<kRouteNpl>(a, (uint32_t)(*memo0 + 1), lv)) set_error(a);
        mx::wave_topk_regs<kRouteNpl>(lv, a.n_experts, a.E, a.norm, rid, rw);
    }
    if constexpr (kLogitRoute) {
        if (bid == 0 && wave == 0 && lane < a.E && a.ids_out) {
            a.ids_out[lane] = rid;
            a.w_out[lane] = rw;
        }
    }

    if (bid < nA) {
        // ================================================= gate / up
        const int s = bid % a.E;
        const int jb = bid / a.E;
        const int j0 = jb * 32;
        const int H = a.H;
        const int hb = H >> 5;                  // 32-blocks per row (64)
        const int bpw = hb >> 2;                // blocks per wave (16)
        const int sa = bpw >> 2;                // K-steps per wave (H/512, <= 4)

        int* memo = reinterpret_cast<int*>(a.ws + kMemoAOff) + s * 32 + jb;
        const int cfg = *reinterpret_cast<const int*>(a.ws + kCfgOff);
        const int launch = *memo;

        const int e = kLogitRoute ? __builtin_amdgcn_readfirstlane(__shfl(rid, s))
                      : ROUTE == ROUTE_DEV_IDS ? __builtin_amdgcn_readfirstlane(a.ids_dev[s]) : pick_id(a, s);
        const uint8_t* gw = a.gate_wp + (int64_t)e * a.wp_stride_gu;
        const uint8_t* gs = a.gate_ws + (int64_t)e * a.ws_stride_gu;
        const uint8_t* uw = a.up_wp + (int64_t)e * a.wp_stride_gu;
        const uint8_t* us = a.up_ws + (int64_t)e * a.ws_stride_gu;

        // weights: 4 row groups (gate lo/hi, up lo/hi) x sa K-steps; step i
        // takes blocks q0 + 4i .. q0 + 4i + 3 of the wave's K quarter (q0 =
        // bpw*wave), lane group g block q0 + 4i + g: the four lanes of a row
        // read 64 contiguous bytes per load (the order of decode_stack.hip)
        uint4 bq[4][4];
        uint32_t bsd[4][4];   // scale dwords of blocks q0 + 4i .. (byte g of dword i)
        const int q0 = bpw * wave;
#pragma unroll
        for (int G = 0; G < 4; ++G) {
            const int row = j0 + 16 * (G & 1) + r;
            const uint8_t* wrow = ((G < 2) ? gw : uw) + (int64_t)row * (H >> 1);
            const uint8_t* srow = ((G < 2) ? gs : us) + (int64_t)row * hb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int blk = q0 + 4 * min(i, sa - 1) + g;
                bq[G][i] = ld_sel(reinterpret_cast<const uint4*>(wrow + blk * 16), i < sa, make_uint4(0, 0, 0, 0));
            }
            if (sa == 4) {   // the quarter's 16 scale bytes in one load (H = 2048)
                const uint4 v = *reinterpret_cast<const uint4*>(srow + q0);
                bsd[G][0] = v.x;
                bsd[G][1] = v.y;
                bsd[G][2] = v.z;
                bsd[G][3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) bsd[G][i] = *reinterpret_cast<const uint32_t*>(srow + q0 + 4 * min(i, sa - 1));
            }
        }

        // x -> three E4M3 terms in LDS (whole row; 8 values per thread)
        if (k0 < H) {
            float v[8];
            const uint32_t w4[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = ROUTE == ROUTE_FUSED ? yf[2 * i] : mx::bf16_to_f32((uint16_t)(w4[i] & 0xFFFFu));
                v[2 * i + 1] = ROUTE == ROUTE_FUSED ? yf[2 * i + 1] : mx::bf16_to_f32((uint16_t)(w4[i] >> 16));
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
        if (threadIdx.x < 2) sm.a.zero[threadIdx.x] = make_uint4(0, 0, 0, 0);
        __syncthreads();

        // MFMA: step i covers blocks {q0 + 4i + gb : gb = 0..3}; A lane group g
        // holds K [16g, +16) and [64 + 16g, +16) of the step, i.e. halves
        // (g & 1) of blocks 4i + (g >> 1) and 4i + 2 + (g >> 1), with block
        // 4i + g's scale.  Operands first, then the MFMAs.  A zero operand is
        // read from the zero region (an address select), not selected after the
        // read: a value select compiles to branches that serialise the LDS reads.
        mx::v8i av[4];
        uint32_t asc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int base = q0 + 4 * min(i, sa - 1);
            const bool ok = r < kTerms && i < sa;
            const uint4* plo = ok ? reinterpret_cast<const uint4*>(&sm.a.x8[rr][(base + (g >> 1)) * 32 + 16 * (g & 1)])
                                  : &sm.a.zero[0];
            const uint4* phi = ok ? reinterpret_cast<const uint4*>(&sm.a.x8[rr][(base + 2 + (g >> 1)) * 32 + 16 * (g & 1)])
                                  : &sm.a.zero[1];
            av[i] = cat8(*plo, *phi);
            const uint32_t c = sm.a.xsc[rr][base + g];
            asc[i] = ok ? c : 127u;
        }
        mx::v4f acc[4];
#pragma unroll
        for (int G = 0; G < 4; ++G) acc[G] = (mx::v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int G = 0; G < 4; ++G)
                acc[G] = mx::mfma16_fp8a_fp4b(av[i], bq[G][i], acc[G], asc[i], (bsd[G][i] >> (8 * g)) & 0xFFu);
#pragma unroll
        for (int G = 0; G < 4; ++G) mx::pin(acc[G]);   // complete the chain before the lane < 16 branch
        // rows 0..2 of D (the three terms) are elements 0..2 of lanes 0..15
        if (lane < 16) {
#pragma unroll
            for (int G = 0; G < 4; ++G) sm.a.red[wave][G][lane] = acc[G][0] + acc[G][1] + acc[G][2];
        }
        __syncthreads();
        // h = silu(g) * u for the 32 rows, one per lane of wave 0, split into
        // E4M3 terms and published as one word per value
        if (wave == 0) {
            const int j = lane & 31;
            float gsum = 0.f, usum = 0.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                gsum += sm.a.red[w][j >> 4][j & 15];
                usum += sm.a.red[w][2 + (j >> 4)][j & 15];
            }
            uint32_t codes;
            const uint32_t bytes = split32(mx::silu_mul_fast(gsum, usum), codes);
            const uint32_t word = bytes | (j < kTerms ? ((codes >> (8 * j)) & 0xFFu) << 24 : 0u);
            const bool cfg_ok = cfg == a.cfg;
            const int64_t w_off = ((int64_t)s * nblk_mi + jb) * kRecWords + j;
            uint32_t* cur = hbuf + (launch & 1) * a.bufwords;
            uint32_t* nxt = hbuf + ((launch & 1) ^ 1) * a.bufwords;
            if (lane < 32 && cfg_ok) {
                __hip_atomic_store(cur + w_off, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(nxt + w_off, kEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (lane == 0) {
                *memo = launch + 1;
                if (!cfg_ok) set_error(a);
            }
        }
        // the launch counts of the router slots, the q|k|v tail, the front
        // and the next layer's attention this launch has no workgroup for
        // move on with it, so a later fused launch agrees (workgroup 0, all
        // threads: one memory round trip)
        if (bid == 0) {
            const int t = threadIdx.x;
            const int nr = ROUTE == ROUTE_FUSED ? a.nr : 0;
            if (t < kMaxRouterWg && t >= nr) reinterpret_cast<int*>(a.ws + kMemoROff)[t] += 1;
            const int nq = ROUTE == ROUTE_FUSED ? a.nq : 0;
            const int nm = ROUTE == ROUTE_FUSED ? a.nm : 0;
            const int no = ROUTE == ROUTE_FUSED ? a.no : 0;
            const int nat = ROUTE == ROUTE_FUSED ? a.nat : 0;
            if (t < kMaxQkvWg && t >= nq) reinterpret_cast<int*>(a.ws + kMemoQOff)[t] += 1;
            if (t < 64 && t >= nm) reinterpret_cast<int*>(a.ws + kMemoMOff)[t] += 1;
            if (t < kMaxOWg && t >= no) reinterpret_cast<int*>(a.ws + kMemoOOff)[t] += 1;
            int* mt = reinterpret_cast<int*>(a.ws + kMemoTOff);
#pragma unroll
            for (int k = t; k < kMaxAttnWg; k += 256)
                if (k >= nat) mt[k] += 1;
        }
        return;
    }

    // ===================================================== down + combine
    const int cb = bid - nA;
    const int c0 = cb * 16;
    const int Mi = a.Mi;
    const int kb = Mi >> 5;          // 32-blocks per down row (24)
    const int steps = (kb + 3) >> 2; // MFMA K-steps (6), <= MS
    int* memo = reinterpret_cast<int*>(a.ws + kMemoBOff) + cb;
    const int cfg = *reinterpret_cast<const int*>(a.ws + kCfgOff);
    const int launch = *memo;
    // wave handles slots 2*wave, 2*wave+1; step i takes blocks 4i .. 4i + 3
    // of the Mi row, lane group g block 4i + g (64 contiguous bytes per row
    // and load; the order of decode_stack.hip)
    int slot[2], eid[2];
    float wgt[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        slot[q] = 2 * wave + q;
        const int sl = slot[q] < a.E ? slot[q] : 0;
        eid[q] = kLogitRoute ? __builtin_amdgcn_readfirstlane(__shfl(rid, sl))
                 : ROUTE == ROUTE_DEV_IDS ? __builtin_amdgcn_readfirstlane(a.ids_dev[sl]) : pick_id(a, sl);
        wgt[q] = kLogitRoute ? __shfl(rw, sl) : ROUTE == ROUTE_DEV_IDS ? a.w_dev[sl] : pick_w(a, sl);
    }
    uint4 bq[2][MS];
    uint32_t bsc[2][MS];   // the scale byte of block 4i + g
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const bool live = slot[q] < a.E;
        const uint8_t* wrow = a.down_wp + (int64_t)eid[q] * a.wp_stride_dn + (int64_t)(c0 + r) * (Mi >> 1);
        const uint8_t* srow = a.down_ws + (int64_t)eid[q] * a.ws_stride_dn + (int64_t)(c0 + r) * kb;
#pragma unroll
        for (int i = 0; i < MS; ++i) {
            const int blk = 4 * i + g;
            bq[q][i] = ld_sel(reinterpret_cast<const uint4*>(wrow + min(blk, kb - 1) * 16),
                              live && i < steps && blk < kb, make_uint4(0, 0, 0, 0));
        }
        if ((kb & 3) == 0) {
#pragma unroll
            for (int i = 0; i < MS; ++i)  // dword i holds blocks 4i .. 4i + 3; past the row: zero data
                bsc[q][i] = (*reinterpret_cast<const uint32_t*>(srow + 4 * min(i, (kb >> 2) - 1)) >> (8 * g)) & 0xFFu;
        } else {  // rows not a dword multiple: byte loads, never past the row
#pragma unroll
            for (int i = 0; i < MS; ++i) {
                const int off = 4 * i + g;
                bsc[q][i] = (live && off < kb) ? (uint32_t)srow[off] : 127u;
            }
        }
    }

    // poll this launch's h words of all slots until none is empty (one probe
    // word first, then every round reloads all of this thread's words: a
    // conditional reload compiles to one wait per word), then unpack the term
    // bytes and codes into LDS.  Thread t owns words 2048k + 8t .. +7 (values
    // 8*(t%4).. of one 32-block).
    const int nwords = a.E * nblk_mi * kRecWords;
    const bool cfg_ok = cfg == a.cfg;
    constexpr int kGroups = (kMaxE * 4 * MS * kRecWords) / 2048;  // groups of 8 words per thread
    const uint32_t* cur = hbuf + (launch & 1) * a.bufwords;
    uint32_t wv[kGroups][8];
    bool ok = cfg_ok;
    if (cfg_ok) {
        int spins = 0;
        const int w0 = min(8 * (64 * wave + 63), nwords - 1);   // one probe word per wave
        uint32_t probe = __hip_atomic_load(cur + w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        while (probe == kEmpty) {
            if (++spins >= kSpinLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(4);
            probe = __hip_atomic_load(cur + w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // 16-byte loads with the agent-scope cache policy (sc1, as the atomic
        // loads use); out-of-range words read as 0 (buffer bounds)
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(cur), (short)0, nwords * 4, 0x00020000);
        while (ok) {
#pragma unroll
            for (int k = 0; k < kGroups; ++k)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const v4u q = __builtin_amdgcn_raw_buffer_load_b128(rs, (2048 * k + 8 * (int)threadIdx.x + 4 * h) * 4, 0, 16);
                    wv[k][4 * h + 0] = q.x;
                    wv[k][4 * h + 1] = q.y;
                    wv[k][4 * h + 2] = q.z;
                    wv[k][4 * h + 3] = q.w;
                }
            bool pending = false;
#pragma unroll
            for (int k = 0; k < kGroups; ++k)
#pragma unroll
                for (int i = 0; i < 8; ++i) pending |= wv[k][i] == kEmpty;
            if (!pending) break;
            if (++spins >= kSpinLimit) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            asm volatile("" ::: "memory");   // the words may change: reload them next round
        }
    }
    if (ok) {
#pragma unroll
        for (int k = 0; k < kGroups; ++k) {
            const int wi = 2048 * k + 8 * (int)threadIdx.x;   // first word; quads never straddle nwords
            if (wi < nwords) {
                const int rec = 64 * k + ((int)threadIdx.x >> 2);   // wi / kRecWords
#pragma unroll
                for (int t = 0; t < kTerms; ++t) {
                    // byte t of words i = 0..7 -> 8 consecutive E4M3 bytes of term t
                    const uint32_t sel = 0x0C0C0000u | ((4u + t) << 8) | (uint32_t)t;
                    const uint32_t lo = __builtin_amdgcn_perm(wv[k][1], wv[k][0], sel) |
                                        (__builtin_amdgcn_perm(wv[k][3], wv[k][2], sel) << 16);
                    const uint32_t hi = __builtin_amdgcn_perm(wv[k][5], wv[k][4], sel) |
                                        (__builtin_amdgcn_perm(wv[k][7], wv[k][6], sel) << 16);
                    *reinterpret_cast<uint64_t*>(sm.b.h8 + (rec * kTerms + t) * 32 + 8 * (threadIdx.x & 3)) =
                        (uint64_t)lo | ((uint64_t)hi << 32);
                }
                if ((threadIdx.x & 3) == 0)
                    sm.b.hsc[rec] = (wv[k][0] >> 24) | ((wv[k][1] >> 24) << 8) | ((wv[k][2] >> 24) << 16);
            }
        }
    }
    if (!ok) set_error(a);
    if (threadIdx.x < 2) sm.b.zero[threadIdx.x] = make_uint4(0, 0, 0, 0);
    if (threadIdx.x == 2) sm.b.code127[0] = 0x7F7F7F7Fu;
    const bool abort = __syncthreads_or(!ok);

    float part = 0.0f;  // this lane's (lane < 16) partial combine over its slots
    if (!abort) {
        bool live[2];
        const uint8_t* h8[2];
        const uint32_t* hsq[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            live[q] = slot[q] < a.E;                                              // wave-uniform
            const int sl = live[q] ? slot[q] : 0;
            h8[q] = sm.b.h8 + (sl * kb * kTerms + rr) * 32;                       // block b at + b*kTerms*32
            hsq[q] = sm.b.hsc + sl * kb;
        }
        // operands of both slots for all steps first (their LDS reads issue
        // back to back), then the two slots' MFMA chains interleaved step by
        // step (independent accumulators).  Zero operands come from the zero
        // region: an address select, no branch between the LDS reads.
        mx::v8i av[2][MS];
        uint32_t asc[2][MS];
#pragma unroll
        for (int i = 0; i < MS; ++i) {
            // step i: B lane group gb holds block 4i + gb (see the gate/up operands)
            const int blo = 4 * i + (g >> 1);
            const int bhi = 4 * i + 2 + (g >> 1);
            const int bown = 4 * i + g;
            const bool rok = r < kTerms && i < steps;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const bool ok = rok && live[q];
                const uint4* plo = (ok && blo < kb) ? reinterpret_cast<const uint4*>(h8[q] + blo * (kTerms * 32) + 16 * (g & 1))
                                                    : &sm.b.zero[0];
                const uint4* phi = (ok && bhi < kb) ? reinterpret_cast<const uint4*>(h8[q] + bhi * (kTerms * 32) + 16 * (g & 1))
                                                    : &sm.b.zero[1];
                const uint32_t* pc = (ok && bown < kb) ? &hsq[q][bown] : &sm.b.code127[0];
                av[q][i] = cat8(*plo, *phi);
                asc[q][i] = (*pc >> (8 * rr)) & 0xFFu;
            }
        }
        mx::v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int i = 0; i < MS; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                acc[q] = mx::mfma16_fp8a_fp4b(av[q][i], bq[q][i], acc[q], asc[q][i], bsc[q][i]);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            mx::pin(acc[q]);
            if (live[q]) part = fmaf(wgt[q], acc[q][0] + acc[q][1] + acc[q][2], part);
        }
    }
    if (lane < 16) sm.b.red[wave][lane] = part;
    __syncthreads();
    if (!abort && threadIdx.x < 16) {
        const int c = c0 + threadIdx.x;
        const float y = sm.b.red[0][threadIdx.x] + sm.b.red[1][threadIdx.x] + sm.b.red[2][threadIdx.x] +
                        sm.b.red[3][threadIdx.x];
        a.out[c] = y;
        if (ROUTE == ROUTE_FUSED && a.nq > 0)   // for the q|k|v tail: (value, this launch's tag)
            __hip_atomic_store(out_words(a) + opos(c),
                               (uint64_t)__float_as_uint(y) | ((uint64_t)(uint32_t)(launch + 1) << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.resid) {
            // runtime/model_runner_v2.py:208: x = x + moe.bfloat16() in bf16
            const float yb = mx::bf16_to_f32(mx::f32_to_bf16_rne(y));
            a.resid[c] = mx::f32_to_bf16_rne(mx::bf16_to_f32(a.x[c]) + yb);
        }
    }
    // the launch count last: a store before a barrier would make the barrier
    // wait for its device-scope acknowledgement
    if (threadIdx.x == 0) *memo = launch + 1;
}

__global__ void reset_workspace_kernel(uint32_t* ws, int cfg, int hwords) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < kHOff / 4) ws[i] = (i == kCfgOff / 4) ? (uint32_t)cfg : 0u;
    if (i < hwords) ws[kHOff / 4 + i] = kEmpty;
    if (i < 2 * kWordsAfterH) ws[kHOff / 4 + hwords + i] = 0u;   // tagged words: tag 0, which no launch uses
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// uint32 words of one h buffer, rounded to 256 bytes
int buf_words(int E, int Mi) { return (int)(align256((size_t)E * (Mi / 32) * kRecWords * 4) / 4); }

}  // namespace

extern "C" size_t mxfp4_decode_layer_workspace_size(int E, int Mi) {
    if (E <= 0 || Mi <= 0) return 0;
    return kHOff + (size_t)2 * buf_words(E, Mi) * 4 + (size_t)kWordsAfterH * 8;
}

extern "C" int mxfp4_decode_layer_reset(void* workspace, int E, int H, int Mi, void* stream) {
    MXH_REQUIRE(workspace, "decode_layer_reset: null workspace");
    MXH_REQUIRE(E >= 1 && E <= kMaxE && Mi >= 32 && Mi <= 1024 && Mi % 32 == 0 && H >= 512 && H <= 2048 && H % 512 == 0,
                "decode_layer_reset: E=%d H=%d Mi=%d out of range", E, H, Mi);
    const int hw = 2 * buf_words(E, Mi);
    const int n = max(max(hw, kHOff / 4), 2 * kWordsAfterH);
    hipLaunchKernelGGL(reset_workspace_kernel, dim3((n + 255) / 256), dim3(256), 0, mxh::as_stream(stream),
                       static_cast<uint32_t*>(workspace), layer_cfg(E, H, Mi), hw);
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

namespace {
// Checks and fills the launch arguments shared by the routing variants.
int layer_args(LayerArgs& a, const void* x, const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
               const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws, int n_experts, int E, int H,
               int Mi, float* out, void* resid_out, void* workspace, size_t workspace_bytes) {
    MXH_REQUIRE(x && gate_wp && gate_ws && up_wp && up_ws && down_wp && down_ws && out && workspace,
                "moe_decode_layer: null pointer");
    MXH_REQUIRE(E >= 1 && E <= kMaxE, "moe_decode_layer: E=%d must be in [1, 8]", E);
    MXH_REQUIRE(n_experts >= E, "moe_decode_layer: n_experts=%d < E=%d", n_experts, E);
    MXH_REQUIRE(H % 512 == 0 && H >= 512 && H <= 2048, "moe_decode_layer: H=%d must be a multiple of 512 in [512, 2048]", H);
    MXH_REQUIRE(Mi % 32 == 0 && Mi >= 32 && Mi <= 1024, "moe_decode_layer: Mi=%d must be a multiple of 32 in [32, 1024]", Mi);
    MXH_REQUIRE(workspace_bytes >= mxfp4_decode_layer_workspace_size(E, Mi), "moe_decode_layer: workspace too small");
    MXH_REQUIRE(((uintptr_t)workspace & 255) == 0, "moe_decode_layer: workspace must be 256-byte aligned");
    MXH_REQUIRE(((uintptr_t)x & 15) == 0, "moe_decode_layer: x must be 16-byte aligned");
    a = LayerArgs{};
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
    a.n_experts = n_experts;
    a.E = E;
    a.H = H;
    a.Mi = Mi;
    a.cfg = layer_cfg(E, H, Mi);
    a.bufwords = buf_words(E, Mi);
    a.out = out;
    a.resid = static_cast<uint16_t*>(resid_out);
    a.ws = static_cast<uint8_t*>(workspace);
    return MXFP4_OK;
}

template <int ROUTE>
int launch_layer(const LayerArgs& a, hipStream_t st) {
    const int nA = a.E * (a.Mi / 32);
    const int nB = a.H / 16;
    const int nR = ROUTE == ROUTE_FUSED ? a.nr : 0;
    const int nQ = ROUTE == ROUTE_FUSED ? a.nq : 0;
    const int nF = ROUTE == ROUTE_FUSED ? a.nm + a.no : 0;
    const int nT = ROUTE == ROUTE_FUSED ? a.nat : 0;
    const int steps = (a.Mi / 32 + 3) / 4;
    const dim3 grid(nF + nR + nA + nB + nQ + nT);
    if (steps <= 6) hipLaunchKernelGGL((decode_layer_kernel<ROUTE, 6>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((decode_layer_kernel<ROUTE, 8>), grid, dim3(256), 0, st, a);
    return mxh::launch_status("moe_decode_layer");
}
}  // namespace

extern "C" int mxfp4_moe_decode_layer(const void* x, const int32_t* ids_host, const float* w_host,
                                      const int32_t* ids_dev, const float* w_dev,
                                      const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
                                      const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws,
                                      int n_experts, int E, int H, int Mi, float* out, void* resid_out,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    LayerArgs a;
    const int rc = layer_args(a, x, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, E, H, Mi, out,
                              resid_out, workspace, workspace_bytes);
    if (rc != MXFP4_OK) return rc;
    MXH_REQUIRE((ids_dev != nullptr) == (w_dev != nullptr), "moe_decode_layer: give ids and weights both on device or both on host");
    MXH_REQUIRE(ids_dev || (ids_host && w_host), "moe_decode_layer: missing routing");
    a.ids_dev = ids_dev;
    a.w_dev = w_dev;
    if (!ids_dev) {
        for (int s = 0; s < E; ++s) {
            MXH_REQUIRE(ids_host[s] >= 0 && ids_host[s] < n_experts, "moe_decode_layer: expert id %d out of range", ids_host[s]);
            a.ids[s] = ids_host[s];
            a.w[s] = w_host[s];
        }
    }
    hipStream_t st = mxh::as_stream(stream);
    return ids_dev ? launch_layer<ROUTE_DEV_IDS>(a, st) : launch_layer<ROUTE_HOST>(a, st);
}

extern "C" int mxfp4_moe_decode_layer_routed(const void* x, const float* logits, int norm, int32_t* ids_out,
                                             float* w_out, const uint8_t* gate_wp, const uint8_t* gate_ws,
                                             const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                                             const uint8_t* down_ws, int n_experts, int E, int H, int Mi,
                                             float* out, void* resid_out, void* workspace, size_t workspace_bytes,
                                             void* stream) {
    LayerArgs a;
    const int rc = layer_args(a, x, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, E, H, Mi, out,
                              resid_out, workspace, workspace_bytes);
    if (rc != MXFP4_OK) return rc;
    MXH_REQUIRE(logits, "moe_decode_layer_routed: null logits");
    MXH_REQUIRE(n_experts <= 64 * kRouteNpl, "moe_decode_layer_routed: n_experts=%d > %d", n_experts, 64 * kRouteNpl);
    MXH_REQUIRE((ids_out != nullptr) == (w_out != nullptr), "moe_decode_layer_routed: give ids_out and w_out both or neither");
    a.logits = logits;
    a.norm = norm ? 1 : 0;
    a.ids_out = ids_out;
    a.w_out = w_out;
    return launch_layer<ROUTE_LOGITS>(a, mxh::as_stream(stream));
}

namespace {
int fused_router_args(LayerArgs& a, const void* x, const float* resid, const void* norm_w, float eps,
                      const uint8_t* router_wp, const uint8_t* router_ws, int norm, void* x_out, void* y_out,
                      float* logits_out, int32_t* ids_out, float* w_out, const uint8_t* gate_wp,
                      const uint8_t* gate_ws, const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                      const uint8_t* down_ws, int n_experts, int E, int H, int Mi, float* out, void* workspace,
                      size_t workspace_bytes) {
    const int rc = layer_args(a, x, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, E, H, Mi, out,
                              nullptr, workspace, workspace_bytes);
    if (rc != MXFP4_OK) return rc;
    MXH_REQUIRE(resid && norm_w && router_wp && router_ws, "moe_decode_layer_fused_router: null pointer");
    MXH_REQUIRE(H == 2048, "moe_decode_layer_fused_router: H=%d (the fused norm is built for 2048)", H);
    MXH_REQUIRE(n_experts % 16 == 0 && n_experts <= 2 * kMaxRouterWg,
                "moe_decode_layer_fused_router: n_experts=%d must be a multiple of 16 up to %d", n_experts,
                2 * kMaxRouterWg);
    MXH_REQUIRE((ids_out != nullptr) == (w_out != nullptr),
                "moe_decode_layer_fused_router: give ids_out and w_out both or neither");
    MXH_REQUIRE(((uintptr_t)resid & 15) == 0 && ((uintptr_t)norm_w & 15) == 0 && ((uintptr_t)router_wp & 15) == 0 &&
                    ((uintptr_t)router_ws & 3) == 0 && ((uintptr_t)x_out & 15) == 0 && ((uintptr_t)y_out & 15) == 0,
                "moe_decode_layer_fused_router: resid, norm_w, router_wp, x_out, y_out must be 16-byte aligned, "
                "router_ws 4-byte");
    a.xres = static_cast<const uint16_t*>(x);
    a.oproj = resid;
    a.nw = static_cast<const uint16_t*>(norm_w);
    a.eps = eps;
    a.rwp = router_wp;
    a.rws = router_ws;
    a.norm = norm ? 1 : 0;
    a.x_out = static_cast<uint16_t*>(x_out);
    a.y_out = static_cast<uint16_t*>(y_out);
    a.logits_out = logits_out;
    a.ids_out = ids_out;
    a.w_out = w_out;
    a.nr = 8 * (n_experts / 16);   // every XCD's copy of the logits
    return MXFP4_OK;
}
}  // namespace

extern "C" int mxfp4_moe_decode_layer_fused_router(const void* x, const float* resid, const void* norm_w, float eps,
                                                   const uint8_t* router_wp, const uint8_t* router_ws, int norm,
                                                   void* x_out, void* y_out, float* logits_out, int32_t* ids_out,
                                                   float* w_out, const uint8_t* gate_wp, const uint8_t* gate_ws,
                                                   const uint8_t* up_wp, const uint8_t* up_ws, const uint8_t* down_wp,
                                                   const uint8_t* down_ws, int n_experts, int E, int H, int Mi,
                                                   float* out, void* workspace, size_t workspace_bytes, void* stream) {
    LayerArgs a;
    const int rc = fused_router_args(a, x, resid, norm_w, eps, router_wp, router_ws, norm, x_out, y_out, logits_out,
                                     ids_out, w_out, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, E,
                                     H, Mi, out, workspace, workspace_bytes);
    if (rc != MXFP4_OK) return rc;
    return launch_layer<ROUTE_FUSED>(a, mxh::as_stream(stream));
}

extern "C" int mxfp4_moe_decode_layer_fused_router_qkv(
    const void* x, const float* resid, const void* norm_w, float eps, const uint8_t* router_wp,
    const uint8_t* router_ws, int norm, void* x_out, void* y_out, float* logits_out, int32_t* ids_out, float* w_out,
    const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp, const uint8_t* up_ws,
    const uint8_t* down_wp, const uint8_t* down_ws, int n_experts, int E, int H, int Mi, const void* qkv_norm_w,
    const uint8_t* qkv_wp, const uint8_t* qkv_ws, int Nq, float* qkv_out, void* x_next_out, float* out,
    void* workspace, size_t workspace_bytes, void* stream) {
    LayerArgs a;
    const int rc = fused_router_args(a, x, resid, norm_w, eps, router_wp, router_ws, norm, x_out, y_out, logits_out,
                                     ids_out, w_out, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, E,
                                     H, Mi, out, workspace, workspace_bytes);
    if (rc != MXFP4_OK) return rc;
    MXH_REQUIRE(qkv_norm_w && qkv_wp && qkv_ws && qkv_out, "moe_decode_layer_fused_router_qkv: null pointer");
    MXH_REQUIRE(Nq >= 1 && Nq <= 64 * kMaxQkvWg, "moe_decode_layer_fused_router_qkv: Nq=%d (1..%d)", Nq,
                64 * kMaxQkvWg);
    MXH_REQUIRE(((uintptr_t)qkv_norm_w & 15) == 0 && ((uintptr_t)qkv_wp & 15) == 0 && ((uintptr_t)qkv_ws & 15) == 0 &&
                    ((uintptr_t)x_next_out & 15) == 0,
                "moe_decode_layer_fused_router_qkv: qkv_norm_w, qkv_wp, qkv_ws, x_next_out must be 16-byte aligned");
    MXH_REQUIRE(!x_next_out || (x_next_out != x && x_next_out != x_out),
                "moe_decode_layer_fused_router_qkv: x_next_out must not alias x or x_out");
    a.qnw = static_cast<const uint16_t*>(qkv_norm_w);
    a.qwp = qkv_wp;
    a.qws = qkv_ws;
    a.qkv_out = qkv_out;
    a.xn_out = static_cast<uint16_t*>(x_next_out);
    a.Nq = Nq;
    a.nq = (Nq + 63) / 64;
    return launch_layer<ROUTE_FUSED>(a, mxh::as_stream(stream));
}

extern "C" int mxfp4_decode_layer_post_attn(
    const void* attn_workspace, size_t attn_workspace_bytes, const int32_t* dpos, int Hq, int max_pos, uint8_t* aq_out, uint8_t* as_out,
    const uint8_t* o_wp, const uint8_t* o_ws, float* oproj_out, const void* x, const void* norm_w, float eps,
    const uint8_t* router_wp, const uint8_t* router_ws, int norm, void* x_out, void* y_out, float* logits_out,
    int32_t* ids_out, float* w_out, const uint8_t* gate_wp, const uint8_t* gate_ws, const uint8_t* up_wp,
    const uint8_t* up_ws, const uint8_t* down_wp, const uint8_t* down_ws, int n_experts, int E, int H, int Mi,
    const void* qkv_norm_w, const uint8_t* qkv_wp, const uint8_t* qkv_ws, int Nq, float* qkv_out, void* x_next_out,
    void* next_attn_workspace, size_t next_attn_workspace_bytes, uint8_t* kvk_next, uint8_t* kvv_next,
    const void* q_norm_next, const void* k_norm_next, int Hkv, float theta, int codec, float* out, void* workspace,
    size_t workspace_bytes, void* stream) {
    MXH_REQUIRE(attn_workspace && dpos && o_wp && o_ws && oproj_out, "decode_layer_post_attn: null pointer");
    MXH_REQUIRE(Hq == kMaxHq, "decode_layer_post_attn: Hq=%d (the o_proj front is built for %d heads of 128)", Hq,
                kMaxHq);
    MXH_REQUIRE(max_pos > 0 && max_pos <= am::kChunk * am::kMaxChunks, "decode_layer_post_attn: max_pos=%d", max_pos);
    MXH_REQUIRE(!aq_out == !as_out, "decode_layer_post_attn: aq_out and as_out go together");
    LayerArgs a;
    int rc = fused_router_args(a, x, oproj_out, norm_w, eps, router_wp, router_ws, norm, x_out, y_out, logits_out,
                               ids_out, w_out, gate_wp, gate_ws, up_wp, up_ws, down_wp, down_ws, n_experts, E, H, Mi,
                               out, workspace, workspace_bytes);
    if (rc != MXFP4_OK) return rc;
    MXH_REQUIRE(H / 16 <= kMaxOWg, "decode_layer_post_attn: H=%d", H);
    MXH_REQUIRE(attn_workspace_bytes >= mxfp4_attn_decode_workspace_size(1, Hq, max_pos),
                "decode_layer_post_attn: attention workspace smaller than mxfp4_attn_decode_workspace_size(1, %d, %d)",
                Hq, max_pos);
    MXH_REQUIRE(((uintptr_t)attn_workspace & 15) == 0 && ((uintptr_t)o_wp & 15) == 0 && ((uintptr_t)o_ws & 15) == 0 &&
                    ((uintptr_t)aq_out & 3) == 0,
                "decode_layer_post_attn: attn_workspace, o_wp, o_ws must be 16-byte aligned, aq_out 4-byte");
    if (qkv_wp) {
        MXH_REQUIRE(qkv_norm_w && qkv_ws && qkv_out, "decode_layer_post_attn: null q|k|v pointer");
        MXH_REQUIRE(Nq >= 1 && Nq <= 64 * kMaxQkvWg, "decode_layer_post_attn: Nq=%d (1..%d)", Nq, 64 * kMaxQkvWg);
        MXH_REQUIRE(((uintptr_t)qkv_norm_w & 15) == 0 && ((uintptr_t)qkv_wp & 15) == 0 &&
                        ((uintptr_t)qkv_ws & 15) == 0 && ((uintptr_t)x_next_out & 15) == 0,
                    "decode_layer_post_attn: qkv_norm_w, qkv_wp, qkv_ws, x_next_out must be 16-byte aligned");
        MXH_REQUIRE(!x_next_out || (x_next_out != x && x_next_out != x_out),
                    "decode_layer_post_attn: x_next_out must not alias x or x_out");
        a.qnw = static_cast<const uint16_t*>(qkv_norm_w);
        a.qwp = qkv_wp;
        a.qws = qkv_ws;
        a.qkv_out = qkv_out;
        a.xn_out = static_cast<uint16_t*>(x_next_out);
        a.Nq = Nq;
        a.nq = (Nq + 63) / 64;
    }
    a.apart = static_cast<const float*>(attn_workspace);
    a.dpos = dpos;
    a.max_pos = max_pos;
    a.nchunk = (max_pos + am::kChunk - 1) / am::kChunk;
    a.aq_out = aq_out;
    a.as_out = as_out;
    a.owp = o_wp;
    a.ows = o_ws;
    a.oproj_out = oproj_out;
    a.nm = Hq;
    a.no = H / 16;
    if (next_attn_workspace) {
        MXH_REQUIRE(qkv_wp, "decode_layer_post_attn: the next layer's attention needs the q|k|v tail");
        MXH_REQUIRE(kvk_next && kvv_next && q_norm_next && k_norm_next, "decode_layer_post_attn: null next-attention pointer");
        MXH_REQUIRE(Hkv >= 1 && Hq == 8 * Hkv && Nq == (Hq + 2 * Hkv) * am::kD,
                    "decode_layer_post_attn: Hkv=%d, Nq=%d (8 query heads per kv head, Nq = (Hq + 2 Hkv) * 128)", Hkv,
                    Nq);
        MXH_REQUIRE(codec == 0 || codec == 1, "decode_layer_post_attn: codec %d", codec);
        MXH_REQUIRE(next_attn_workspace_bytes >= mxfp4_attn_decode_workspace_size(1, Hq, max_pos) &&
                        ((uintptr_t)next_attn_workspace & 15) == 0 && next_attn_workspace != attn_workspace,
                    "decode_layer_post_attn: next attention workspace (16-byte aligned, "
                    "mxfp4_attn_decode_workspace_size bytes, not attn_workspace)");
        MXH_REQUIRE(((uintptr_t)kvk_next & 15) == 0 && ((uintptr_t)kvv_next & 3) == 0,
                    "decode_layer_post_attn: kv cache rows must be aligned");
        MXH_REQUIRE(a.nchunk * Hkv <= kMaxAttnWg, "decode_layer_post_attn: max_pos=%d x Hkv=%d too large", max_pos, Hkv);
        a.apart_n = static_cast<float*>(next_attn_workspace);
        a.kvk_n = kvk_next;
        a.kvv_n = kvv_next;
        a.qn_n = static_cast<const uint16_t*>(q_norm_next);
        a.kn_n = static_cast<const uint16_t*>(k_norm_next);
        a.theta = theta;
        a.codec = codec;
        a.hkv = Hkv;
        a.nat = a.nchunk * Hkv;
    }
    return launch_layer<ROUTE_FUSED>(a, mxh::as_stream(stream));
}
