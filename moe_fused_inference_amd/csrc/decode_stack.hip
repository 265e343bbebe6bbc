// decode_stack.hip -- a run of consecutive decode MoE layers for one token in
// one launch (batch 1).
//
// Computes, for layers l = 0 .. L-1 of a stack,
//     y_l     = sum_s w[l][s] * down_e(silu(gate_e(x_l)) * up_e(x_l)),  e = ids[l][s]
//     x_{l+1} = bf16(x_l + bf16(y_l))
// -- the reference's per-layer MoE step (runtime/model_runner_v2.py:185-208,
// kernels src/ext/mxfp4_decode.cu:24-50,177-299) applied layer after layer,
// on un-quantized bf16 activations in fp32 with exactly the arithmetic of the
// one-layer kernel (decode_layer.hip), so the results equal chained one-layer
// launches bit for bit.  The routing of every layer (ids, w) is an input, so
// layer l+1's expert weights stream while layer l is still being computed.
//
// Placement.  MI355X has 8 XCDs of 32 CUs, each XCD with its own L2, and
// deals the workgroups of a 256-workgroup grid to the XCDs round-robin, 32
// each; a workgroup takes a CU.  Slot s of the top-E routing lives on XCD s
// (read from the XCC id register).  The XCD's workgroups j = blockIdx.x / 8
// form two sets by the parity of j, and set p computes the layers l with
// l % 2 == p: while one set runs a layer's hand-offs the other set streams
// the weights of its next layer into registers.  A poll from a CU comes back
// only after the loads that CU already has in flight (measured: a same-XCD
// hand-off takes ~0.23 us on a CU with nothing in flight and ~3 us behind a
// layer's worth of prefetch, while streaming on other CUs costs it nothing),
// so a workgroup issues the loads of its next layer (l+2) only after the last
// poll of layer l.  Within its set, workgroup jj = j / 2 (0..15) takes the
// gate/up row tiles jj, jj+16, jj+32, .. of the slot's 2*Mi/16 tiles (gate
// tiles first) and the down rows (output columns) [jj*H/16, (jj+1)*H/16).
//
// One layer, per workgroup; each of its four waves owns a quarter of the
// gate/up K range and a share of every other step:
//   1. x_l: poll this XCD's copy of x_l (bf16, published by the other set in
//      the previous layer) for the wave's K quarter; E4M3 terms into LDS;
//   2. gate/up MFMAs; the four waves' partial sums meet in LDS; publish the
//      raw g or u values of the workgroup's tiles (fp32);
//   3. poll the slot's g/u for the wave's share of the 32-blocks of h;
//      h = silu(g) * u and its E4M3 terms into LDS (barrier: all of h);
//   4. down MFMAs on the wave's column tiles; publish y_s per column (fp32);
//   5. poll y_t of every slot t for the wave's share of the workgroup's
//      columns; y = sum_t w_t y_t (the one-layer kernel's order), x_{l+1} =
//      bf16(x_l + bf16(y)); publish x_{l+1} for those columns into this XCD's
//      copy;
//   6. barrier, then issue the weight loads of layer l+2.
// Every XCD computes all of x_{l+1}, so the x and g/u hand-offs stay inside
// one L2 (plain stores, agent-scope loads that hit the local L2) and only the
// per-slot y crosses XCDs (fan-in of 8 producers per consumer).  With STRICT
// a layer's loads are issued only once the wave has x_l: the timing of
// routing that depends on x.
//
// Hand-off words.  Every published value travels in a 64-bit word (value,
// tag), written and read as one single-copy-atomic access; the tag is the
// layer count (a memo per (slot, j) in the workspace, read at entry, + L at
// exit; all workgroups agree on it), never 0.  A consumer waits until every
// word carries the expected tag, so no buffer is ever emptied and no store
// completion is ever waited for.  Two buffers per kind, used by alternate
// layers, suffice: a producer writes layer c+2 into the buffer of layer c
// only after it has (transitively) seen every consumer of layer c finish.
//
// Co-residency.  The 256 workgroups must be resident at once (each waits on
// others of every layer): each takes more than half of a CU's LDS, so a CU
// holds one, and the host refuses the launch unless the occupancy query
// allows the whole grid on a 256-CU device.  Every wait is bounded
// (kSpinLimit polls); on expiry, or when another workgroup has set the error
// flag, a wave stops waiting, the results are garbage and the flag stays set
// until the workspace is reset.
#include "decode_common.h"
#include "lds_dma.h"
#include "mx_host.h"

namespace {

using namespace dl;

constexpr int kXcds = 8;              // XCDs = slots
constexpr int kPerXcd = 32;           // CUs (workgroups) per XCD
constexpr int kPerSet = kPerXcd / 2;  // workgroups per set (two sets, alternate layers)
constexpr int kGrid = kXcds * kPerXcd;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxNT = 8;             // gate/up tiles per workgroup (Mi <= 1024)
static_assert(kMaxNT <= 2 * kWaves, "the g/u publish takes at most two tiles per wave");
constexpr int kLdsLayers = 128;       // layers whose routing and weight pointers are staged in LDS
constexpr int kRecBytes = 112;        // LDS record of 32 values: 3 x 32 term bytes, codes at 96..98

// workspace layout (bytes)
constexpr int kCfgOff = 0;            // int32 config word written by reset
constexpr int kErrOff = 256;          // int32 error flag
constexpr int kMemoOff = 1024;        // int32 layer count per workgroup
constexpr int kBufOff = kMemoOff + 4 * kGrid;
constexpr int kNBuf = 2;              // buffers per kind, alternate layers

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
    int gu_q, part_q, x_q;      // 64-bit words per XCD (g/u, x) / per slot (y) of one buffer
    int64_t buf_q;              // 64-bit words of one buffer (all kinds, all XCDs)
    uint8_t* ws;
};

__host__ __device__ constexpr int stack_cfg(int E, int H, int Mi) {
    return 0x5D000000 | (E << 16) | ((H / 512) << 12) | (Mi / 32);
}

// 64-bit words of one buffer: g/u (2*Mi per XCD), y (H per slot), x (H per XCD)
__host__ __device__ constexpr int gu_words(int Mi) { return ((2 * Mi + 31) / 32) * 32; }
__host__ __device__ constexpr int part_words(int H) { return ((H + 31) / 32) * 32; }
__host__ __device__ constexpr int x_words(int H) { return ((H + 31) / 32) * 32; }
__host__ __device__ constexpr int64_t buf_words(int H, int Mi) {
    return (int64_t)kXcds * (gu_words(Mi) + part_words(H) + x_words(H));
}

struct Route {                                   // rows read as 16-byte words
    alignas(16) int32_t ids[kLdsLayers];           // this slot's expert per layer
    alignas(16) float w[kLdsLayers][kMaxE];        // every slot's combine weight per layer
    alignas(16) const uint8_t* ptr[kLdsLayers][6];  // the layer's six stacked weight pointers
};

union Smem {
    struct {
        uint4 zero[2];
        uint32_t code127[4];
        uint8_t xr[64 * kRecBytes];             // x_l in E4M3 terms, 32-value records (H/32 <= 64)
        uint8_t hr[32 * kRecBytes];             // h_l in E4M3 terms (Mi/32 <= 32)
        uint16_t xb[2048];                      // x_l in bf16 (the combine's residual)
        float hs[1024];                         // h_l (fp32), split source
        float red[kWaves][kMaxNT][16];          // gate/up partial sums: wave x tile x row
        Route rt;
    } s;
    uint8_t one_per_cu[84 * 1024];              // more than half of a CU's LDS: one workgroup per CU
};
constexpr int kSinkOff = 80 * 1024;             // strict prefetch: LDS sink of 256 bytes, past Smem::s
static_assert(sizeof(decltype(Smem::s)) <= kSinkOff, "the prefetch sink lies past the kernel's LDS data");

// Error flag bits: a bounded wait expired, the workspace belongs to another shape.
constexpr int kErrWait = 1, kErrCfg = 2;

__device__ __forceinline__ void set_error(const StackArgs& a, int bits = kErrWait) {
    __hip_atomic_fetch_or(reinterpret_cast<int*>(a.ws + kErrOff), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool error_set(const StackArgs& a) {
    return __hip_atomic_load(reinterpret_cast<const int*>(a.ws + kErrOff), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// A wave-uniform pointer held in SGPRs (buffer descriptors must be uniform).
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const uint8_t* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(uniform_ptr(p)), (short)0, bytes, 0x00020000);
}

// Loads of the read-only routing arrays and layer table through the
// constant address space (scalar loads) for layers past the LDS copy.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p, int i) {
    typedef const __attribute__((address_space(4))) T* cptr;
    return ((cptr)(uintptr_t)p)[i];
}

// Workgroup barrier for LDS only: waits for this wave's LDS operations, not
// for its outstanding global loads (__syncthreads' release fence would wait
// for the next layer's weight prefetch).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Publish / poll of (value, tag) words.  Publishing to this XCD's L2 only
// (consumers on the same XCD) is a plain store; to the device (consumers on
// other XCDs) an agent-scope store, written through to the coherence point.
// Polls are agent-scope loads: they see a line dirty in the local L2 and
// fetch anything else from the coherence point.
__device__ __forceinline__ void put_local(uint64_t* p, uint32_t value, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void put_device(uint64_t* p, uint32_t value, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A whole 64-bit word (lo, hi) to this XCD's L2.
__device__ __forceinline__ void put_word(uint64_t* p, uint32_t lo, uint32_t hi) {
    __hip_atomic_store(p, ((uint64_t)hi << 32) | lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The 16-bit tag of a layer count's x words: 1..65535, never 0 (the reset
// value); two layer counts two apart (the previous use of a buffer) differ.
__device__ __forceinline__ uint32_t tag16(uint32_t tag) { return tag % 65535u + 1u; }

typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// Bounded poll of N 64-bit words per lane -- byte offsets off[i] of the region
// of descriptor rs, lanes with ok[i] false take nothing -- until each carries
// `tag` in bits 32 + TSH and up; w[i] = the words.  Agent-scope 8-byte loads
// (single-copy atomic: value and tag always come from the same store).  `live`
// false (an earlier wait failed): one load, no wait.  Returns false on expiry
// or when the error flag is set.
template <int N, int TSH = 0>
__device__ __forceinline__ bool poll_words(const StackArgs& a, __amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[N],
                                           const bool (&ok)[N], uint32_t tag, v2u (&w)[N], bool live) {
    int spins = 0;
    while (true) {
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = __builtin_amdgcn_raw_buffer_load_b64(rs, off[i], 0, 16);
        bool pending = false;
#pragma unroll
        for (int i = 0; i < N; ++i) pending |= ok[i] && (w[i].y >> TSH) != tag;
        if (!live) return false;
        if (__builtin_amdgcn_ballot_w64(pending) == 0) return true;   // the wave polls as one
        if (++spins >= kSpinLimit || ((spins & 255) == 0 && error_set(a))) return false;
        __builtin_amdgcn_s_sleep(1);
        asm volatile("" ::: "memory");   // the words may change: reload them next round
    }
}

// poll_words with 16-byte loads: load i (byte offset off[i], 16-byte aligned)
// brings words w[2i] and w[2i+1], each single-copy atomic on its own.
template <int N, int TSH = 0>
__device__ __forceinline__ bool poll_pairs(const StackArgs& a, __amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[N],
                                           const bool (&ok)[N], uint32_t tag, v2u (&w)[2 * N], bool live) {
    int spins = 0;
    while (true) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rs, off[i], 0, 16);
            w[2 * i] = v2u{v.x, v.y};
            w[2 * i + 1] = v2u{v.z, v.w};
        }
        bool pending = false;
#pragma unroll
        for (int i = 0; i < N; ++i) pending |= ok[i] && ((w[2 * i].y >> TSH) != tag || (w[2 * i + 1].y >> TSH) != tag);
        if (!live) return false;
        if (__builtin_amdgcn_ballot_w64(pending) == 0) return true;   // the wave polls as one
        if (++spins >= kSpinLimit || ((spins & 255) == 0 && error_set(a))) return false;
        __builtin_amdgcn_s_sleep(1);
        asm volatile("" ::: "memory");   // the words may change: reload them next round
    }
}

// poll_words for (value, 32-bit tag) words: v[i] = the values
template <int N>
__device__ __forceinline__ bool poll_tagged(const StackArgs& a, __amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[N],
                                            const bool (&ok)[N], uint32_t tag, uint32_t (&v)[N], bool live) {
    v2u w[N];
    const bool r = poll_words<N>(a, rs, off, ok, tag, w, live);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = w[i].x;
    return r;
}

// Word position of column col's x word within the XCD's x buffer: inside each
// 256-column block, column 4 j + c sits at 128 (c >> 1) + 2 j + (c & 1), so the
// x poll of lane j (columns 4 j .. 4 j + 3 of a block) is two lane-contiguous
// 16-byte loads, each bringing two of its columns (8 cache lines a load).  A
// permutation of each block (H is a multiple of 512).
__device__ __forceinline__ int xpos(int col) {
    return (col & ~255) | ((col & 2) << 6) | (((col >> 2) & 63) << 1) | (col & 1);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t region(const uint64_t* p, int words) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(p), (short)0, words * 8, 0x00020000);
}

// Splits 8 consecutive values (a quarter of a 32-block; the 4 lanes of a quad
// hold one block) into the LDS record layout: term t's bytes at
// rec + 32t + `pos`, the block's codes at rec + 96 + t (written by the quad's
// first lane).  Same arithmetic as split8 everywhere else.
__device__ __forceinline__ void split8_to_record(float v[8], uint8_t* rec, int pos) {
    uint64_t w8[kTerms];
    uint32_t codes;
    split8(v, w8, codes);
#pragma unroll
    for (int t = 0; t < kTerms; ++t) {
        *reinterpret_cast<uint64_t*>(rec + 32 * t + pos) = w8[t];
        if ((threadIdx.x & 3) == 0) rec[96 + t] = (uint8_t)(codes >> (8 * t));
    }
}

__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 16)" : "=s"(v));
    return v & 0xFu;
}

// NT: gate/up tiles per workgroup (Mi/128 rounded up to even); MS: down K
// steps bound; KB4: Mi/32 a multiple of 4 (down scale bytes in aligned dwords).
template <bool STRICT, int MS, bool KB4, int NT>
__global__ __launch_bounds__(kThreads, 1) void decode_stack_kernel(StackArgs a) {
    __shared__ __align__(16) Smem smu;
    auto& sm = smu.s;

    const int lane = threadIdx.x & 63;
    const int cw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave 0..3
    const int r = lane & 15;
    const int g = lane >> 4;
    const int rr = r < kTerms ? r : 0;
    const int bid = blockIdx.x;
    // The dispatcher deals workgroups to the 8 XCDs round-robin, but the XCD
    // of workgroup 0 varies between dispatches (it follows the previous
    // dispatch in a graph replay), so the slot is the XCD this workgroup runs
    // on, and bid / 8 numbers the 32 workgroups of each XCD.  (Were the deal
    // not a rotation, a (slot, j) pair would go missing and the bounded waits
    // on its outputs would set the error flag.)
    const int s = (int)__builtin_amdgcn_readfirstlane(xcc_id());   // slot = XCD
    const int j = bid / kXcds;                 // workgroup within the XCD
    const int par = j & 1;                     // its set: layers l with l % 2 == par
    const int jj = j >> 1;                     // workgroup within the set
    const int L = a.n_layers;
    const int E = a.E;
    const int H = a.H;
    const int Mi = a.Mi;
    if (s >= E) return;                        // no slot on this XCD
    int* memo = reinterpret_cast<int*>(a.ws + kMemoOff) + s * kPerXcd + j;
    const uint32_t c0 = (uint32_t)__builtin_amdgcn_readfirstlane(*memo);
    const bool cfg_ok = *reinterpret_cast<const int*>(a.ws + kCfgOff) == a.cfg;
    if (!cfg_ok) {
        if (threadIdx.x == 0) set_error(a, kErrCfg);
        return;
    }
    uint64_t* bufs = reinterpret_cast<uint64_t*>(a.ws + kBufOff);
    // kind bases within buffer b: g/u of XCD s, y of slot t, x of XCD s
    auto gu_base = [&](int b) { return bufs + b * a.buf_q + (int64_t)s * a.gu_q; };
    auto part_base = [&](int b, int t) { return bufs + b * a.buf_q + (int64_t)kXcds * a.gu_q + (int64_t)t * a.part_q; };
    auto x_base = [&](int b) {
        return bufs + b * a.buf_q + (int64_t)kXcds * (a.gu_q + a.part_q) + (int64_t)s * a.x_q;
    };

    // routing and weight pointers of the first kLdsLayers layers
    {
        const int nl = min(L, kLdsLayers);
        for (int i = threadIdx.x; i < nl * kMaxE; i += kThreads) {
            const int l = i / kMaxE, k = i % kMaxE;
            sm.rt.w[l][k] = k < E ? a.w[l * E + k] : 0.0f;
        }
        for (int i = threadIdx.x; i < nl; i += kThreads) sm.rt.ids[i] = a.ids[i * E + s];
        for (int i = threadIdx.x; i < nl * 6; i += kThreads)
            sm.rt.ptr[i / 6][i % 6] = reinterpret_cast<const uint8_t* const*>(a.layers)[i];
        if (threadIdx.x < 2) sm.zero[threadIdx.x] = make_uint4(0, 0, 0, 0);
        if (threadIdx.x == 2) sm.code127[0] = 0x7F7F7F7Fu;
        __syncthreads();
    }
    // layer l's six weight pointers and this slot's expert: from LDS with three 16-byte reads
    // under one wave-uniform branch (a select per field compiles to a branch and an LDS
    // round trip each, ~0.3 us per layer in series)
    struct LayerRoute {
        const uint8_t* p[6];
        int e;
    };
    auto route = [&](int l) -> LayerRoute {
        LayerRoute r;
        int e;
        if (l < kLdsLayers) {
            const uint4* q = reinterpret_cast<const uint4*>(&sm.rt.ptr[l][0]);
            const uint4 v[3] = {q[0], q[1], q[2]};
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                r.p[2 * k] = reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)v[k].y << 32) | v[k].x));
                r.p[2 * k + 1] = reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)v[k].w << 32) | v[k].z));
            }
            e = sm.rt.ids[l];
        } else {
#pragma unroll
            for (int k = 0; k < 6; ++k) r.p[k] = ld_const(reinterpret_cast<const uint8_t* const*>(a.layers), 6 * l + k);
            e = ld_const(a.ids, l * E + s);
        }
        e = __builtin_amdgcn_readfirstlane(e);
        r.e = e < 0 ? 0 : (e >= a.n_experts ? a.n_experts - 1 : e);   // memory safety only
        return r;
    };

    const int hb = H >> 5;                     // 32-blocks along H
    const int ntile = Mi >> 3;                 // gate + up tiles of 16 rows (2*Mi/16)
    const int ncol = H >> 4;                   // down and combine columns per workgroup
    const int c0d = jj * ncol;
    const int nct = ncol >> 4;                 // down column tiles per workgroup (1..8)
    const int kb = Mi >> 5;                    // 32-blocks along Mi
    const int steps = (kb + 3) >> 2;           // down K steps

    // ---- gate/up weights: K quarter cw (blocks q0 = bpw*cw ..) of tiles jj + 16m.
    // MFMA step i takes blocks q0 + 4i .. q0 + 4i + 3, lane group g block
    // q0 + 4i + g: the four lanes of a row read 64 contiguous bytes per load
    // (with lane group g on blocks q0 + sa*g + i, 16-byte pieces 64 bytes
    // apart, a set's per-layer burst took twice as long).  Offsets of tiles
    // past the last are out of the descriptor's range: their loads return
    // zeros without touching memory.
    constexpr uint32_t kNone = 0x80000000u;
    const int bpw = hb >> 2;
    const int sa = bpw >> 2;
    const int q0 = bpw * cw;
    uint4 bq[NT][4];
    uint32_t bs[NT][4];   // scale dwords of blocks q0 + 4i .. q0 + 4i + 3 (byte g of dword i)
    uint32_t woff[NT], soff[NT];
    bool tup[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) {
        const int t = jj + kPerSet * m;
        const bool ok = t < ntile;
        tup[m] = t >= (ntile >> 1);
        const int row = 16 * (tup[m] ? t - (ntile >> 1) : t) + r;
        woff[m] = ok ? (uint32_t)(row * (H >> 1) + (q0 + g) * 16) : kNone;
        soff[m] = ok ? (uint32_t)(row * hb + q0) : kNone;
    }
    // valid = false: a zero-extent descriptor, so the loads return zeros
    // without touching memory
    auto load_gu = [&](const LayerRoute& rt, bool valid) {
        const int e = rt.e;
        const int wbytes = valid ? Mi * (H >> 1) : 0, sbytes = valid ? Mi * hb : 0;
        const __amdgpu_buffer_rsrc_t rw[2] = {rsrc(rt.p[0] + (int64_t)e * a.wp_stride_gu, wbytes),
                                              rsrc(rt.p[1] + (int64_t)e * a.wp_stride_gu, wbytes)};
        const __amdgpu_buffer_rsrc_t rs[2] = {rsrc(rt.p[3] + (int64_t)e * a.ws_stride_gu, sbytes),
                                              rsrc(rt.p[4] + (int64_t)e * a.ws_stride_gu, sbytes)};
#pragma unroll
        for (int m = 0; m < NT; ++m) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rw[tup[m]], woff[m] + 64 * min(i, sa - 1), 0, 0);
                bq[m][i] = make_uint4(v.x, v.y, v.z, v.w);
            }
            if (sa == 4) {   // the quarter's 16 scale bytes in one load (H = 2048)
                const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rs[tup[m]], soff[m], 0, 0);
                bs[m][0] = v.x;
                bs[m][1] = v.y;
                bs[m][2] = v.z;
                bs[m][3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    bs[m][i] = __builtin_amdgcn_raw_buffer_load_b32(rs[tup[m]], soff[m] + 4 * min(i, sa - 1), 0, 0);
            }
        }
    };
    // STRICT: the gate/up rows load_gu would read, touched with 4-byte LDS-DMA
    // loads into a sink (no registers held, nothing the compiler waits on), so
    // the lines come into this XCD's L2 for the workgroup of the other set
    // that computes the layer
    auto prefetch_gu = [&](const LayerRoute& rt) {
        const int e = rt.e;
        const uint32_t sink = __builtin_amdgcn_readfirstlane(mx::lds_addr(smu.one_per_cu + kSinkOff));
        const mx::v4u rw[2] = {mx::buf_rsrc(rt.p[0] + (int64_t)e * a.wp_stride_gu, (int64_t)Mi * (H >> 1)),
                               mx::buf_rsrc(rt.p[1] + (int64_t)e * a.wp_stride_gu, (int64_t)Mi * (H >> 1))};
        const mx::v4u rs[2] = {mx::buf_rsrc(rt.p[3] + (int64_t)e * a.ws_stride_gu, (int64_t)Mi * hb),
                               mx::buf_rsrc(rt.p[4] + (int64_t)e * a.ws_stride_gu, (int64_t)Mi * hb)};
#pragma unroll
        for (int m = 0; m < NT; ++m) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < sa) mx::dma4(woff[m] + 64 * i, tup[m] ? rw[1] : rw[0], 0, sink);
            mx::dma4(soff[m], tup[m] ? rs[1] : rs[0], 0, sink);
        }
    };
    // ---- down weights: column tiles cw and cw + 4 (16 columns each) of the
    // workgroup's columns.  Step i takes blocks 4i .. 4i + 3 of the Mi row,
    // lane group g block 4i + g (64 contiguous bytes per row and load);
    // blocks past the row reload its last block (finite data, valid scale)
    // against zero activations.
    bool dok[2];
    uint32_t woffd[2], soffd[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int ct = cw + 4 * k;
        dok[k] = ct < nct;
        const int drow = c0d + 16 * ct + r;
        woffd[k] = dok[k] ? (uint32_t)(drow * (Mi >> 1)) : kNone;
        soffd[k] = dok[k] ? (uint32_t)(drow * kb) : kNone;
    }
    uint4 dq[2][MS];
    uint32_t dsc[2][MS];   // scale byte of block 4i + g (KB4: its dword, byte g)
    auto load_dn = [&](const LayerRoute& rt, bool valid) {
        const int e = rt.e;
        const __amdgpu_buffer_rsrc_t rw = rsrc(rt.p[2] + (int64_t)e * a.wp_stride_dn, valid ? H * (Mi >> 1) : 0);
        const __amdgpu_buffer_rsrc_t rs = rsrc(rt.p[5] + (int64_t)e * a.ws_stride_dn, valid ? H * kb : 0);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
#pragma unroll
            for (int i = 0; i < MS; ++i) {
                const v4u q = __builtin_amdgcn_raw_buffer_load_b128(rw, woffd[k] + 16 * min(4 * i + g, kb - 1), 0, 0);
                dq[k][i] = make_uint4(q.x, q.y, q.z, q.w);
            }
            if (KB4 && kb == 4 * MS) {
                // the row's MS scale dwords are contiguous: 16-byte loads and an 8-byte tail
                // (fewer load instructions in the layer's burst)
#pragma unroll
                for (int i = 0; i + 4 <= MS; i += 4) {
                    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rs, soffd[k] + 4 * i, 0, 0);
                    dsc[k][i] = v.x, dsc[k][i + 1] = v.y, dsc[k][i + 2] = v.z, dsc[k][i + 3] = v.w;
                }
#pragma unroll
                for (int i = MS & ~3; i + 2 <= MS; i += 2) {
                    const v2u v = __builtin_amdgcn_raw_buffer_load_b64(rs, soffd[k] + 4 * i, 0, 0);
                    dsc[k][i] = v.x, dsc[k][i + 1] = v.y;
                }
                if (MS & 1) dsc[k][MS - 1] = __builtin_amdgcn_raw_buffer_load_b32(rs, soffd[k] + 4 * (MS - 1), 0, 0);
            } else {
#pragma unroll
                for (int i = 0; i < MS; ++i) {
                    if (KB4) dsc[k][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, soffd[k] + 4 * min(i, (kb >> 2) - 1), 0, 0);
                    else dsc[k][i] = __builtin_amdgcn_raw_buffer_load_b8(rs, soffd[k] + min(4 * i + g, kb - 1), 0, 0);
                }
            }
        }
    };

    if (!STRICT) {
        const LayerRoute rt = route(min(par, L - 1));
        load_dn(rt, par < L);
        load_gu(rt, par < L);
    }
    bool live = true;
    for (int l = par; l < L; l += 2) {
        const uint32_t tag = c0 + (uint32_t)l + 1u;          // this layer's tag (never 0)
        const int b = (int)((c0 + (uint32_t)l) % kNBuf);
        if (STRICT && l >= 1) {
            // the other set computes layer l-1 now: once x_{l-1} is complete
            // (that layer's routing known) this workgroup pulls its partner's
            // gate/up rows of layer l-1 (the workgroup of the same index in
            // the other set, on this XCD) into their L2, so the partner's own
            // loads of them, issued after its down rows, find them there
            const int m = l - 1;
            if (m >= 1) {
                const int bm = (int)((c0 + (uint32_t)m) % kNBuf);
                const __amdgpu_buffer_rsrc_t rs = region(x_base((bm + kNBuf - 1) % kNBuf), H);
                const int nq = H >> 2;
                const int q0 = cw * nq;
                uint32_t off[4];
                bool ok[4];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        ok[2 * i + j] = 256 * i + 4 * lane < nq;
                        off[2 * i + j] = (uint32_t)(xpos(q0 + min(256 * i + 4 * lane, nq - 4) + 2 * j) * 8);
                    }
                v2u xw[8];
                live = poll_pairs<4, 16>(a, rs, off, ok, tag16(c0 + (uint32_t)m), xw, live);
            }
            prefetch_gu(route(m));
        }
        // combine weights of every slot (read now, used after the y poll)
        float wt[kMaxE];
        if (l < kLdsLayers) {   // two 16-byte reads (the LDS copy holds 0 for t >= E)
            const float4 w0 = *reinterpret_cast<const float4*>(&sm.rt.w[l][0]);
            const float4 w1 = *reinterpret_cast<const float4*>(&sm.rt.w[l][4]);
            wt[0] = w0.x, wt[1] = w0.y, wt[2] = w0.z, wt[3] = w0.w;
            wt[4] = w1.x, wt[5] = w1.y, wt[6] = w1.z, wt[7] = w1.w;
        } else {
#pragma unroll
            for (int t = 0; t < kMaxE; ++t) wt[t] = t < E ? ld_const(a.w, l * E + t) : 0.0f;
        }
        // ---- 1. x_l for the wave's K quarter (columns cw*H/4 ..) into E4M3 term records (LDS)
        // and, for the combine, bf16 (LDS)
        {
            const int nq = H >> 2;                  // columns per quarter (128..512)
            const int q0 = cw * nq;
            if (l == 0) {
                // the launch's input: split here, lane -> values q0 + 8 lane .. +7 (whole quads)
                if (8 * lane < nq) {
                    const int k0 = q0 + 8 * lane;
                    const uint4 q = *reinterpret_cast<const uint4*>(a.x0 + k0);
                    *reinterpret_cast<uint4*>(&sm.xb[k0]) = q;
                    const uint32_t xq[4] = {q.x, q.y, q.z, q.w};
                    float v[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[2 * i] = mx::bf16_to_f32((uint16_t)(xq[i] & 0xFFFFu));
                        v[2 * i + 1] = mx::bf16_to_f32((uint16_t)(xq[i] >> 16));
                    }
                    split8_to_record(v, sm.xr + (k0 >> 5) * kRecBytes, k0 & 31);
                }
            } else {
                // published (already split) in layer l-1 by the other set: one word per column,
                // [term bytes 0..2 | code of term (column % 32) for columns 0..2 of a block |
                //  bf16 | tag16] at word xpos(column); lane -> columns q0 + 256 i + 4 lane .. +3
                const __amdgpu_buffer_rsrc_t rs = region(x_base((b + kNBuf - 1) % kNBuf), H);
                uint32_t off[4];
                bool ok[4];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {   // columns 2j, 2j+1 of the lane's four (adjacent words)
                        ok[2 * i + j] = 256 * i + 4 * lane < nq;
                        off[2 * i + j] = (uint32_t)(xpos(q0 + min(256 * i + 4 * lane, nq - 4) + 2 * j) * 8);
                    }
                v2u xw[8];   // xw[4 i + c]: column c of the lane's four in group i
                live = poll_pairs<4, 16>(a, rs, off, ok, tag16(tag - 1u), xw, live);
                // byte selects (v_perm_b32: selector byte k < 4 takes byte k of the second
                // operand, 4..7 byte k - 4 of the first, 0x0c a zero): columns 0, 1 and 2, 3
                // interleaved first, then term t's four bytes, the block's codes and the bf16 pairs
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    if (256 * i + 4 * lane < nq) {
                        const int c0 = q0 + 256 * i + 4 * lane;
                        uint8_t* rec = sm.xr + (c0 >> 5) * kRecBytes;
                        const uint32_t w0 = xw[4 * i].x, w1 = xw[4 * i + 1].x, w2 = xw[4 * i + 2].x, w3 = xw[4 * i + 3].x;
                        const uint32_t q01 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);   // w0.0 w1.0 w0.1 w1.1
                        const uint32_t q23 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
                        const uint32_t r01 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);   // w0.2 w1.2 w0.3 w1.3
                        const uint32_t r23 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
                        *reinterpret_cast<uint32_t*>(rec + (c0 & 31)) = __builtin_amdgcn_perm(q23, q01, 0x05040100u);
                        *reinterpret_cast<uint32_t*>(rec + 32 + (c0 & 31)) = __builtin_amdgcn_perm(q23, q01, 0x07060302u);
                        *reinterpret_cast<uint32_t*>(rec + 64 + (c0 & 31)) = __builtin_amdgcn_perm(r23, r01, 0x05040100u);
                        if ((c0 & 31) == 0)   // codes of terms 0..2: byte 3 of the block's columns 0..2
                            *reinterpret_cast<uint32_t*>(rec + 96) = __builtin_amdgcn_perm(r23, r01, 0x0c060302u);
                        *reinterpret_cast<uint2*>(&sm.xb[c0]) =
                            make_uint2(__builtin_amdgcn_perm(xw[4 * i + 1].y, xw[4 * i].y, 0x05040100u),
                                       __builtin_amdgcn_perm(xw[4 * i + 3].y, xw[4 * i + 2].y, 0x05040100u));
                    }
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's own records, read below
        }
        if (STRICT) {
            const LayerRoute rt = route(l);
            load_dn(rt, true);
            load_gu(rt, true);
        }
        // ---- 2. gate/up MFMAs: A = x_l terms (rows 0..2), B = the tile's weight rows
        {
            mx::v8i av[4];
            uint32_t asc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // step i, blocks q0 + 4i + gb: A lane group g holds K [16g, +16) and [64 + 16g, +16) of
                // the step, i.e. halves (g & 1) of blocks 4i + (g >> 1) and 4i + 2 + (g >> 1); its scale is
                // block 4i + g's
                const int base = q0 + 4 * min(i, sa - 1);
                const bool ok = r < kTerms && i < sa;
                const uint4* plo = ok ? reinterpret_cast<const uint4*>(sm.xr + (base + (g >> 1)) * kRecBytes + 32 * rr + 16 * (g & 1))
                                      : &sm.zero[0];
                const uint4* phi = ok ? reinterpret_cast<const uint4*>(sm.xr + (base + 2 + (g >> 1)) * kRecBytes + 32 * rr + 16 * (g & 1))
                                      : &sm.zero[1];
                av[i] = cat8(*plo, *phi);
                const uint32_t c = sm.xr[(base + g) * kRecBytes + 96 + rr];
                asc[i] = ok ? c : 127u;
            }
            // K step outer, tiles inner, held in that order (sched_barrier): NT independent
            // accumulations in flight.  Left to itself the scheduler emits each tile's four
            // steps back to back, and a dependent MFMA waits out its predecessor (~60 clocks
            // issue to issue against ~37 for independent ones)
            mx::v4f acc[NT];
#pragma unroll
            for (int m = 0; m < NT; ++m) acc[m] = (mx::v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int m = 0; m < NT; ++m)
                    acc[m] = mx::mfma16_fp8a_fp4b(av[i], bq[m][i], acc[m], asc[i], (bs[m][i] >> (8 * g)) & 0xFFu);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int m = 0; m < NT; ++m) mx::pin(acc[m]);
            if (lane < 16) {
#pragma unroll
                for (int m = 0; m < NT; ++m) sm.red[cw][m][lane] = acc[m][0] + acc[m][1] + acc[m][2];
            }
        }
        lds_barrier();                                                   // B2: gate/up partial sums
        // publish the g/u values of tiles cw and cw + 4 in one pass: lane 16 i + r = row r of
        // tile cw + 4 i (NT <= 8: at most two tiles per wave)
        {
            const int m = cw + kWaves * (lane >> 4);
            const int t = jj + kPerSet * m;
            if (lane < 32 && m < NT && t < ntile) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) v += sm.red[w][m][lane & 15];
                put_local(gu_base(b) + t * 16 + (lane & 15), __float_as_uint(v), tag);
            }
        }
        // ---- 3. the slot's g/u for this wave's 32-blocks of h (rows r0 .. r0 + nr), row 64k + lane
        // of them per load (coalesced); h = silu(g) * u per row into LDS; then lane 8i + q -> rows
        // 4q .. 4q+3 of block i into E4M3 term records (8 lanes per block)
        {
            const int bph = (kb + 3) >> 2;                // blocks per wave (<= 8)
            const int blo = min(cw * bph, kb), bhi = min(blo + bph, kb);
            const int r0 = 32 * blo, nr = 32 * (bhi - blo);
            const __amdgpu_buffer_rsrc_t rs = region(gu_base(b), 2 * Mi);
            // KG groups of 64 rows: bph <= MS blocks, so nr <= 32 MS rows
            constexpr int KG = (MS + 1) / 2;
            uint32_t off[2 * KG];
            bool ok[2 * KG];
            uint32_t gv[2 * KG];
#pragma unroll
            for (int k = 0; k < KG; ++k) {
                const int row = r0 + min(64 * k + lane, max(nr - 1, 0));
                ok[k] = ok[KG + k] = 64 * k + lane < nr;
                off[k] = (uint32_t)(min(row, Mi - 1) * 8);
                off[KG + k] = (uint32_t)((Mi + min(row, Mi - 1)) * 8);
            }
            live = poll_tagged<2 * KG>(a, rs, off, ok, tag, gv, live);
#pragma unroll
            for (int k = 0; k < KG; ++k) {
                const float h = mx::silu_mul_fast(__uint_as_float(gv[k]), __uint_as_float(gv[KG + k]));
                if (64 * k < nr && ok[k]) sm.hs[r0 + 64 * k + lane] = h;   // 64k < nr: wave-uniform
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's own h values, read below
            const int hblk = blo + (lane >> 3);
            if (hblk < bhi) {
                const int pos = 4 * (lane & 7);
                const uint4 q = *reinterpret_cast<const uint4*>(&sm.hs[32 * hblk + pos]);
                float v[4] = {__uint_as_float(q.x), __uint_as_float(q.y), __uint_as_float(q.z), __uint_as_float(q.w)};
                uint32_t w4[kTerms], codes;
                split4(v, w4, codes);
                uint8_t* rec = sm.hr + hblk * kRecBytes;
#pragma unroll
                for (int t = 0; t < kTerms; ++t) *reinterpret_cast<uint32_t*>(rec + 32 * t + pos) = w4[t];
                if (pos == 0) *reinterpret_cast<uint32_t*>(rec + 96) = codes;
            }
        }
        lds_barrier();                                                   // B3: h_l staged
        // ---- 4. down MFMAs: A = h_l terms, B = 16 columns' down rows (two column tiles, their
        // accumulations interleaved); publish y_s
        {
            const uint8_t* h8 = sm.hr + 32 * rr;   // term rr of block 0
            // all A operands first, then the two tiles' steps interleaved and held in that
            // order (sched_barrier), as for gate/up
            mx::v8i av[MS];
            uint32_t asc[MS];
#pragma unroll
            for (int i = 0; i < MS; ++i) {
                // step i, blocks 4i + gb (see the gate/up operands)
                const int blo = 4 * i + (g >> 1);
                const int bhi = 4 * i + 2 + (g >> 1);
                const int bown = 4 * i + g;
                const bool rok = r < kTerms && i < steps;
                const uint4* plo = (rok && blo < kb) ? reinterpret_cast<const uint4*>(h8 + blo * kRecBytes + 16 * (g & 1))
                                                     : &sm.zero[0];
                const uint4* phi = (rok && bhi < kb) ? reinterpret_cast<const uint4*>(h8 + bhi * kRecBytes + 16 * (g & 1))
                                                     : &sm.zero[1];
                const uint8_t* pc = (rok && bown < kb) ? sm.hr + bown * kRecBytes + 96 + rr
                                                       : reinterpret_cast<const uint8_t*>(&sm.code127[0]);
                av[i] = cat8(*plo, *phi);
                asc[i] = *pc;
            }
            mx::v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int i = 0; i < MS; ++i) {
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const uint32_t bsc = KB4 ? (dsc[k][i] >> (8 * g)) & 0xFFu : dsc[k][i] & 0xFFu;
                    acc[k] = mx::mfma16_fp8a_fp4b(av[i], dq[k][i], acc[k], asc[i], bsc);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            // both tiles' sums before either (conditional) store: with a sum inside the store's
            // branch the compiler sinks the second tile's MFMA chain behind the first store
            float ysum[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                mx::pin(acc[k]);
                ysum[k] = acc[k][0] + acc[k][1] + acc[k][2];
            }
#pragma unroll
            for (int k = 0; k < 2; ++k)
                if (dok[k] && lane < 16)
                    put_device(part_base(b, s) + c0d + 16 * (cw + 4 * k) + lane, __float_as_uint(ysum[k]), tag);
        }
        // ---- 5. y of every slot for block cb = 4 jj + cw (lanes 0..31 = its columns); x_{l+1};
        // its E4M3 terms, published with the bf16 value for the other set's next layer
        {
            const int cb = 4 * jj + cw;
            if (cb < hb) {
                const bool ccol = lane < 32;
                const int col = 32 * cb + (lane & 31);
                // slot t's y at word t*part_q + col of the y region; lanes 0..31 poll slots
                // 0..3 and lanes 32..63 slots 4..7 of the same 32 columns (four loads a lane)
                static_assert(kMaxE == 8, "the y poll splits the slots over the two wave halves");
                const int hf = lane >> 5;
                const __amdgpu_buffer_rsrc_t rs = region(part_base(b, 0), E * a.part_q);
                uint32_t off[4];
                bool ok[4];
                uint32_t yv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int t = 4 * hf + j;
                    ok[j] = t < E;
                    off[j] = (uint32_t)((min(t, E - 1) * a.part_q + col) * 8);
                }
                live = poll_tagged<4>(a, rs, off, ok, tag, yv, live);
                // the one-layer kernel's order: per slot pair (2w, 2w+1) a fused
                // multiply-add chain from 0, then the four pair sums left to right;
                // pairs 2, 3 come from the upper half (permlane32 swap: lane i < 32
                // reads lane i + 32 in element 1)
                float pr[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int t0 = 4 * hf + 2 * u;
                    const float w0 = hf ? wt[4 + 2 * u] : wt[2 * u], w1 = hf ? wt[5 + 2 * u] : wt[1 + 2 * u];
                    float part = 0.0f;
                    if (t0 < E) part = fmaf(w0, __uint_as_float(yv[2 * u]), part);
                    if (t0 + 1 < E) part = fmaf(w1, __uint_as_float(yv[2 * u + 1]), part);
                    pr[u] = part;
                }
                const auto up0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(pr[0]), __float_as_uint(pr[0]), false, false);
                const auto up1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(pr[1]), __float_as_uint(pr[1]), false, false);
                float y = pr[0];
                y = y + pr[1];
                y = y + __uint_as_float(up0[1]);
                y = y + __uint_as_float(up1[1]);
                // runtime/model_runner_v2.py:208: x = x + moe.bfloat16() in bf16
                const float yb = mx::bf16_to_f32(mx::f32_to_bf16_rne(y));
                const uint16_t xn = mx::f32_to_bf16_rne(mx::bf16_to_f32(sm.xb[col]) + yb);
                if (l + 1 < L) {
                    uint32_t codes;
                    const uint32_t bytes = split32(mx::bf16_to_f32(xn), codes);   // over lanes 0..31
                    const uint32_t code = (lane & 31) < kTerms ? (codes >> (8 * (lane & 31))) & 0xFFu : 0u;
                    if (ccol) put_word(x_base(b) + xpos(col), bytes | (code << 24), (uint32_t)xn | (tag16(tag) << 16));
                } else if (s == 0 && ccol) {
                    a.x_out[col] = xn;
                }
                if (s == 0 && ccol) {
                    if (a.x_all) a.x_all[(int64_t)l * H + col] = xn;
                    if (a.y_all) a.y_all[(int64_t)l * H + col] = y;
                }
            }
        }
        lds_barrier();                                                   // B5: every poll of the layer done
        if (!STRICT) {
            // layer l+2 streams while the other set computes layer l+1
            const LayerRoute rt = route(l + 2 < L ? l + 2 : l);
            load_dn(rt, l + 2 < L);
            load_gu(rt, l + 2 < L);
        }
    }
    if (!live) set_error(a);
    if (threadIdx.x == 0) *memo = (int)(c0 + (uint32_t)L);
}

__global__ void reset_stack_kernel(uint32_t* ws, int cfg, int64_t words) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < kBufOff / 4) ws[i] = (i == kCfgOff / 4) ? (uint32_t)cfg : 0u;
    if (i < words) ws[kBufOff / 4 + i] = 0u;   // tag 0: no layer
}

}  // namespace

extern "C" size_t mxfp4_decode_stack_workspace_size(int E, int H, int Mi) {
    if (E <= 0 || H <= 0 || Mi <= 0) return 0;
    return kBufOff + (size_t)kNBuf * (size_t)buf_words(H, Mi) * 8;
}

extern "C" int mxfp4_decode_stack_reset(void* workspace, int E, int H, int Mi, void* stream) {
    MXH_REQUIRE(workspace, "decode_stack_reset: null workspace");
    MXH_REQUIRE(E >= 1 && E <= kMaxE && Mi >= 32 && Mi <= 1024 && Mi % 32 == 0 && H >= 512 && H <= 2048 && H % 512 == 0,
                "decode_stack_reset: E=%d H=%d Mi=%d out of range", E, H, Mi);
    const int64_t words = (int64_t)kNBuf * buf_words(H, Mi) * 2;   // uint32 words of the buffers
    const int64_t n = words > kBufOff / 4 ? words : kBufOff / 4;
    hipLaunchKernelGGL(reset_stack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, mxh::as_stream(stream),
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

namespace {
template <bool ST, int MS, bool K4>
const void* stack_kernel_nt(int nt) {
    switch (nt) {
        case 2: return reinterpret_cast<const void*>(&decode_stack_kernel<ST, MS, K4, 2>);
        case 4: return reinterpret_cast<const void*>(&decode_stack_kernel<ST, MS, K4, 4>);
        case 6: return reinterpret_cast<const void*>(&decode_stack_kernel<ST, MS, K4, 6>);
        default: return reinterpret_cast<const void*>(&decode_stack_kernel<ST, MS, K4, 8>);
    }
}
template <bool ST>
const void* stack_kernel(int ms, bool k4, int nt) {
    if (ms <= 6) return k4 ? stack_kernel_nt<ST, 6, true>(nt) : stack_kernel_nt<ST, 6, false>(nt);
    return k4 ? stack_kernel_nt<ST, 8, true>(nt) : stack_kernel_nt<ST, 8, false>(nt);
}
}  // namespace

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
    int dev = 0, n_cu = 0;
    MXH_REQUIRE(hipGetDevice(&dev) == hipSuccess &&
                    hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess,
                "moe_decode_stack: cannot query the CU count");
    MXH_REQUIRE(n_cu == kGrid, "moe_decode_stack: needs a GPU of %d CUs in %d XCDs (this one has %d CUs)", kGrid, kXcds,
                n_cu);
    const int steps = (Mi / 32 + 3) / 4;
    const bool kb4 = (Mi / 32) % 4 == 0;
    const int nt = (((Mi / 8 + kPerSet - 1) / kPerSet) + 1) & ~1;   // gate/up tiles per workgroup, even
    const void* kern = strict ? stack_kernel<true>(steps, kb4, nt) : stack_kernel<false>(steps, kb4, nt);
    int per_cu = 0;
    MXH_REQUIRE(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, 0) == hipSuccess,
                "moe_decode_stack: occupancy query failed");
    // every workgroup waits on others, so the whole grid must be resident at once
    MXH_REQUIRE((int64_t)per_cu * n_cu >= kGrid,
                "moe_decode_stack: %d workgroups but only %d x %d can be resident at once", kGrid, per_cu, n_cu);
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
    a.gu_q = gu_words(Mi);
    a.part_q = part_words(H);
    a.x_q = x_words(H);
    a.buf_q = buf_words(H, Mi);
    a.ws = static_cast<uint8_t*>(workspace);
    void* args[] = {&a};
    const hipError_t le = hipLaunchKernel(kern, dim3(kGrid), dim3(kThreads), args, 0, mxh::as_stream(stream));
    if (le != hipSuccess) {
        mxh::set_error("moe_decode_stack: kernel launch failed: %s", hipGetErrorString(le));
        (void)hipGetLastError();
        return (int)le;
    }
    return mxh::launch_status("moe_decode_stack");
}
