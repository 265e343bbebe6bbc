// step_ops.hip -- the non-MoE ops of a decode step, so a whole Qwen3-MoE
// decode step runs on this library's kernels (the reference's loop,
// runtime/model_runner_v2.py:130-217 forward_decode and :220-300
// forward_batch, driven as in runtime/decode_v2.py:64-71):
//
//   embed_rows_kernel      embedding gather with MXFP4 row dequant
//                          (runtime/weight_store.py:47-65 dequant_rows_gpu):
//                          bf16(sign * E2M1 magnitude * 2^(code-127)), exact.
//   norm_quant_kernel      optional residual add x = bf16(x + bf16(o)), then
//                          RMSNorm (runtime/model_runner.py:20-25: fp32
//                          mean of squares, rsqrt, cast back to bf16, times
//                          the bf16 weight) and the MXFP4 quantization of the
//                          normed row (prequant, bit-exact) in one pass.
//   qk_rope_kv_kernel      per token: q/k head RMSNorm on the fp32 projections
//                          (the reference's q_norm / k_norm, result rounded to
//                          bf16), half-layout RoPE (runtime/model_runner.py:
//                          28-41, fp32 products, bf16 result), q out as bf16,
//                          k and bf16(v) written as E4M3 KV bytes at row
//                          dpos + m, in the decode extension's kv_write codec
//                          (src/ext/mxfp4_decode.cu:437-489, the graph
//                          runner's write, runtime/model_runner_v3.py:98-101)
//                          or in torch's float8_e4m3fn conversion (the batch
//                          step's, runtime/model_runner_v2.py:256-257).
//   argmax_kernel          greedy next token per row (logits[m].argmax(),
//                          first maximum; runtime/decode_v2.py:71) over
//                          slices of the row, and the position dpos += M,
//                          both on the device, so a captured step graph can
//                          be replayed step after step.
#include "head_rope.h"
#include "kv_codec.h"
#include "mx_device.h"
#include "mx_host.h"

namespace {

// ------------------------------------------------------------------ embedding
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint8_t* __restrict__ wp, const uint8_t* __restrict__ ws,
                                                         int K, int Kp, const int32_t* __restrict__ ids, int V,
                                                         uint16_t* __restrict__ out) {
    const int m = blockIdx.y;
    const int k0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (k0 >= K) return;
    int id = ids[m];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);   // memory safety only
    const uint32_t nib = *reinterpret_cast<const uint32_t*>(wp + (int64_t)id * (Kp / 2) + k0 / 2);
    const uint32_t code = ws[(int64_t)id * (Kp / 32) + k0 / 32];
    // 2^(code-127) as fp32 (codes 0 and 255 never need a denormal or NaN here:
    // code 0 -> 2^-127 is denormal, built exactly from its bits)
    const float scale = code > 0u ? __uint_as_float(code << 23) : __uint_as_float(0x00400000u);
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = mx::e2m1_value((nib >> (8 * i)) & 15u) * scale;
        const float b = mx::e2m1_value((nib >> (8 * i + 4)) & 15u) * scale;
        o[i] = (uint32_t)mx::f32_to_bf16_rne(a) | ((uint32_t)mx::f32_to_bf16_rne(b) << 16);
    }
    uint16_t* dst = out + (int64_t)m * K + k0;
    if (k0 + 8 <= K) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
        for (int i = 0; i < 8 && k0 + i < K; ++i) dst[i] = (uint16_t)(o[i / 2] >> (16 * (i & 1)));
    }
}

// ------------------------------------------------------------------ RMSNorm + quantize
// Sum over the 256 threads of a workgroup (4 waves): DPP/shuffle inside the
// wave, then LDS across waves.  Deterministic order.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = mx::wave_sum_butterfly(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();   // red may still be read by a previous call
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup per row; H <= 256 * 8 * kMaxIt.  Thread t owns elements
// 8t + 2048 i (i < H/2048), so a 32-block is 4 consecutive threads.
constexpr int kMaxIt = 4;

template <bool RESID>
__global__ __launch_bounds__(256) void norm_quant_kernel(const uint16_t* __restrict__ x, const float* __restrict__ o,
                                                         const uint16_t* __restrict__ w, float eps, int H,
                                                         uint16_t* __restrict__ x_out, uint16_t* __restrict__ y,
                                                         uint8_t* __restrict__ yq, uint8_t* __restrict__ ys) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const int64_t rb = (int64_t)m * H;
    const int nit = H / 2048;
    float v[kMaxIt][8];
    uint4 wv[kMaxIt];   // the norm weight, loaded with x rather than after the reduction
    float ss = 0.0f;
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
        if (it < nit) {
            const int k0 = 8 * threadIdx.x + 2048 * it;
            wv[it] = *reinterpret_cast<const uint4*>(w + k0);
            const uint4 q = *reinterpret_cast<const uint4*>(x + rb + k0);
            const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[it][2 * i] = mx::bf16_to_f32((uint16_t)(wq[i] & 0xFFFFu));
                v[it][2 * i + 1] = mx::bf16_to_f32((uint16_t)(wq[i] >> 16));
            }
            if (RESID) {
                // runtime/model_runner_v2.py:185/208: x = x + o.bfloat16() (bf16 add)
                const float4 a = *reinterpret_cast<const float4*>(o + rb + k0);
                const float4 b = *reinterpret_cast<const float4*>(o + rb + k0 + 4);
                const float of[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                uint32_t xo[4];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float ob = mx::bf16_to_f32(mx::f32_to_bf16_rne(of[i]));
                    v[it][i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(v[it][i] + ob));
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xo[i] = (uint32_t)mx::f32_to_bf16_rne(v[it][2 * i]) | ((uint32_t)mx::f32_to_bf16_rne(v[it][2 * i + 1]) << 16);
                *reinterpret_cast<uint4*>(x_out + rb + k0) = make_uint4(xo[0], xo[1], xo[2], xo[3]);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = fmaf(v[it][i], v[it][i], ss);
        }
    }
    const float var = block_sum(ss, red) / (float)H;
    const float r = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int it = 0; it < kMaxIt; ++it) {
        if (it < nit) {
            const int k0 = 8 * threadIdx.x + 2048 * it;
            const uint32_t wq[4] = {wv[it].x, wv[it].y, wv[it].z, wv[it].w};
            float yv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float wi = mx::bf16_to_f32((uint16_t)(wq[i / 2] >> (16 * (i & 1))));
                const float t = mx::bf16_to_f32(mx::f32_to_bf16_rne(v[it][i] * r));   // (xf * r).to(bf16)
                yv[i] = mx::bf16_to_f32(mx::f32_to_bf16_rne(t * wi));                 // * weight, bf16
            }
            uint32_t yo[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                yo[i] = (uint32_t)mx::f32_to_bf16_rne(yv[2 * i]) | ((uint32_t)mx::f32_to_bf16_rne(yv[2 * i + 1]) << 16);
            *reinterpret_cast<uint4*>(y + rb + k0) = make_uint4(yo[0], yo[1], yo[2], yo[3]);
            // MXFP4 of the normed row (quant/fp4_format.py): block amax over the
            // 4 threads of the 32-block, E8M0 code, E2M1 nibbles
            float am = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(yv[i]));
            am = fmaxf(am, __shfl_xor(am, 1));
            am = fmaxf(am, __shfl_xor(am, 2));
            const uint32_t code = mx::e8m0_code(am);
            const uint32_t nib = mx::e2m1_pack8(yv, mx::e8m0_inv_scale(code));
            *reinterpret_cast<uint32_t*>(yq + (int64_t)m * (H / 2) + k0 / 2) = nib;
            if ((threadIdx.x & 3) == 0) ys[(int64_t)m * (H / 32) + k0 / 32] = (uint8_t)code;
        }
    }
}

// ------------------------------------------------------------------ q/k norm + RoPE + KV write
constexpr int kD = 128;

// Workgroup (token m, 4 heads): wave w handles head 4*blockIdx.y + w of the
// Hq + Hkv + Hkv (q, k, v) heads of the fused projection row; lane l owns
// elements l and l + 64 of a head, which are the RoPE partners (D = 128, half
// layout).
__global__ __launch_bounds__(256) void qk_rope_kv_kernel(const float* __restrict__ qkv, const uint16_t* __restrict__ qw,
                                                         const uint16_t* __restrict__ kw, float eps, float theta,
                                                         const int32_t* __restrict__ dpos, int Hq, int Hkv,
                                                         uint16_t* __restrict__ q_out, uint8_t* __restrict__ kvk,
                                                         uint8_t* __restrict__ kvv, int max_pos, int codec) {
    const int m = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nh = Hq + 2 * Hkv;
    const int h = blockIdx.y * 4 + wave;
    if (h >= nh) return;
    const int pos = *dpos + m;
    const float* row = qkv + (int64_t)m * nh * kD;
    const float2 cs = hr::rope_cs(theta, lane, pos);
    {
        const float a = row[h * kD + lane], b = row[h * kD + lane + 64];
        if (h >= Hq + Hkv) {   // v: bf16, then the KV byte
            const int hv = h - Hq - Hkv;
            if (pos >= 0 && pos < max_pos) {
                uint8_t* dst = kvv + ((int64_t)pos * Hkv + hv) * kD;
                dst[lane] = (uint8_t)kv::e4m3_encode(mx::bf16_to_f32(mx::f32_to_bf16_rne(a)), codec);
                dst[lane + 64] = (uint8_t)kv::e4m3_encode(mx::bf16_to_f32(mx::f32_to_bf16_rne(b)), codec);
            }
            return;
        }
        const uint16_t* nw = h < Hq ? qw : kw;
        uint16_t ba, bb;
        hr::norm_rope(a, b, mx::bf16_to_f32(nw[lane]), mx::bf16_to_f32(nw[lane + 64]), eps, cs, ba, bb);
        if (h < Hq) {
            uint16_t* dst = q_out + ((int64_t)m * Hq + h) * kD;
            dst[lane] = ba;
            dst[lane + 64] = bb;
        } else if (pos >= 0 && pos < max_pos) {
            uint8_t* dst = kvk + ((int64_t)pos * Hkv + (h - Hq)) * kD;
            dst[lane] = (uint8_t)kv::e4m3_encode(mx::bf16_to_f32(ba), codec);
            dst[lane + 64] = (uint8_t)kv::e4m3_encode(mx::bf16_to_f32(bb), codec);
        }
    }
}

// ------------------------------------------------------------------ greedy argmax
// Workgroup (slice p of kArgSlice logits, row m): the first index of the
// slice's maximum (NaNs never win) goes to the workspace; the workgroup that
// finishes a row last (a counter per row) merges the row's slices, and the
// one that finishes the last row advances dpos.  Every counter is put back
// to zero by the workgroup that read it last, so the workspace needs one
// zero fill when it is allocated and never again (graph replays included).
constexpr int kArgPer = 16;                  // logits per thread
constexpr int kArgSlice = 256 * kArgPer;     // logits per workgroup

struct ArgWs {
    uint32_t* cnt;   // (M) slices done per row, then 1 word: rows done
    float* val;      // (M, P) slice maxima
    int32_t* idx;    // (M, P) their indices
};

__device__ __forceinline__ void arg_better(float& best, int& idx, float ob, int oi) {
    if (ob > best || (ob == best && oi < idx)) {
        best = ob;
        idx = oi;
    }
}

__device__ __forceinline__ void arg_wave(float& best, int& idx) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) arg_better(best, idx, __shfl_xor(best, o), __shfl_xor(idx, o));
}

__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ logits, int V, int M,
                                                     int32_t* __restrict__ ids, int32_t* __restrict__ dpos,
                                                     ArgWs ws) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    __shared__ int last;
    const int p = blockIdx.x, m = blockIdx.y, P = gridDim.x;
    const float* row = logits + (int64_t)m * V;
    const int base = p * kArgSlice;
    // thread t holds logits base + 4 (i * 256 + t) + j, i < 4, j < 4: a
    // float4 per i, all four loads issued before any is used
    float v[kArgPer];
    const bool vec = (V & 3) == 0;   // 16-byte aligned rows
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = base + 4 * (i * 256 + threadIdx.x);
        if (vec && e + 4 <= V) {
            const float4 f = *reinterpret_cast<const float4*>(row + e);
            v[4 * i] = f.x;
            v[4 * i + 1] = f.y;
            v[4 * i + 2] = f.z;
            v[4 * i + 3] = f.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[4 * i + j] = e + j < V ? row[e + j] : -INFINITY;
        }
    }
    float best = -INFINITY;
    int idx = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = base + 4 * (i * 256 + threadIdx.x) + j;
            if (v[4 * i + j] > best) {   // strictly greater: indices rise along the scan
                best = v[4 * i + j];
                idx = e;
            }
        }
    arg_wave(best, idx);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) arg_better(best, idx, bv[w], bi[w]);
        ws.val[(int64_t)m * P + p] = best;
        ws.idx[(int64_t)m * P + p] = idx;
        __threadfence();
        const uint32_t done = __hip_atomic_fetch_add(&ws.cnt[m], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = done == (uint32_t)(P - 1);
    }
    __syncthreads();
    if (!last || wave != 0) return;
    // the row's last workgroup: merge its P slices (wave 0)
    const int lane = threadIdx.x & 63;
    best = -INFINITY;
    idx = 0x7FFFFFFF;
    for (int q = lane; q < P; q += 64)
        arg_better(best, idx, __hip_atomic_load(&ws.val[(int64_t)m * P + q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                   __hip_atomic_load(&ws.idx[(int64_t)m * P + q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    arg_wave(best, idx);
    if (lane == 0) {
        ids[m] = idx == 0x7FFFFFFF ? 0 : idx;
        __hip_atomic_store(&ws.cnt[m], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (dpos) {
            __threadfence();
            const uint32_t rows = __hip_atomic_fetch_add(&ws.cnt[M], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            if (rows == (uint32_t)(M - 1)) {
                *dpos += M;
                __hip_atomic_store(&ws.cnt[M], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

size_t argmax_ws_bytes(int M, int V) {
    const int64_t P = (V + kArgSlice - 1) / kArgSlice;
    const int64_t head = ((int64_t)(M + 1) * 4 + 255) / 256 * 256;
    return (size_t)(head + 2 * (int64_t)M * P * 4);
}

}  // namespace

extern "C" int mxfp4_embed_rows(const uint8_t* wp, const uint8_t* ws, int V, int K, const int32_t* ids, int M,
                                void* out, void* stream) {
    MXH_REQUIRE(wp && ws && ids && out, "embed_rows: null pointer");
    MXH_REQUIRE(V > 0 && K > 0 && K % 8 == 0 && M > 0 && M <= 65535, "embed_rows: V=%d K=%d M=%d (K a multiple of 8)", V, K, M);
    MXH_REQUIRE(((uintptr_t)out & 15) == 0, "embed_rows: out must be 16-byte aligned");
    const int Kp = (K + 31) / 32 * 32;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((K / 8 + 255) / 256, M), dim3(256), 0, mxh::as_stream(stream), wp, ws, K,
                       Kp, ids, V, static_cast<uint16_t*>(out));
    return mxh::launch_status("embed_rows");
}

extern "C" int mxfp4_rmsnorm_quant(const void* x, const float* resid, const void* w, float eps, int M, int H,
                                   void* x_out, void* y, uint8_t* yq, uint8_t* ys, void* stream) {
    MXH_REQUIRE(x && w && y && yq && ys, "rmsnorm_quant: null pointer");
    MXH_REQUIRE(M > 0 && H > 0 && H % 2048 == 0 && H <= 2048 * kMaxIt, "rmsnorm_quant: M=%d H=%d (H a multiple of 2048, <= %d)", M,
                H, 2048 * kMaxIt);
    MXH_REQUIRE(!resid || x_out, "rmsnorm_quant: a residual needs x_out");
    MXH_REQUIRE((((uintptr_t)x | (uintptr_t)w | (uintptr_t)y | (uintptr_t)resid | (uintptr_t)x_out) & 15) == 0,
                "rmsnorm_quant: x, w, y, resid, x_out must be 16-byte aligned");
    hipStream_t st = mxh::as_stream(stream);
    if (resid)
        hipLaunchKernelGGL(norm_quant_kernel<true>, dim3(M), dim3(256), 0, st, static_cast<const uint16_t*>(x), resid,
                           static_cast<const uint16_t*>(w), eps, H, static_cast<uint16_t*>(x_out),
                           static_cast<uint16_t*>(y), yq, ys);
    else
        hipLaunchKernelGGL(norm_quant_kernel<false>, dim3(M), dim3(256), 0, st, static_cast<const uint16_t*>(x),
                           nullptr, static_cast<const uint16_t*>(w), eps, H, nullptr, static_cast<uint16_t*>(y), yq, ys);
    return mxh::launch_status("rmsnorm_quant");
}

extern "C" int mxfp4_qk_norm_rope_kv(const float* qkv, const void* q_norm_w, const void* k_norm_w, float eps,
                                     float theta, const int32_t* dpos, int M, int Hq, int Hkv, int D, void* q_out,
                                     uint8_t* kvk, uint8_t* kvv, int max_pos, int codec, void* stream) {
    MXH_REQUIRE(qkv && q_norm_w && k_norm_w && dpos && q_out && kvk && kvv, "qk_norm_rope_kv: null pointer");
    MXH_REQUIRE(codec == 0 || codec == 1, "qk_norm_rope_kv: codec %d (0 kv_write's, 1 torch float8_e4m3fn)", codec);
    MXH_REQUIRE(D == kD, "qk_norm_rope_kv: D=%d (the reference's kernels assume 128)", D);
    MXH_REQUIRE(M > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && max_pos > 0, "qk_norm_rope_kv: M=%d Hq=%d Hkv=%d max_pos=%d", M,
                Hq, Hkv, max_pos);
    hipLaunchKernelGGL(qk_rope_kv_kernel, dim3(M, (Hq + 2 * Hkv + 3) / 4), dim3(256), 0, mxh::as_stream(stream), qkv,
                       static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w), eps, theta, dpos,
                       Hq, Hkv, static_cast<uint16_t*>(q_out), kvk, kvv, max_pos, codec);
    return mxh::launch_status("qk_norm_rope_kv");
}

extern "C" size_t mxfp4_argmax_workspace_size(int M, int V) {
    if (M <= 0 || V <= 0) return 0;
    return argmax_ws_bytes(M, V);
}

extern "C" int mxfp4_argmax_advance(const float* logits, int M, int V, int32_t* ids, int32_t* dpos, void* ws,
                                    size_t ws_bytes, void* stream) {
    MXH_REQUIRE(logits && ids && ws, "argmax_advance: null pointer");
    MXH_REQUIRE(M > 0 && M <= 65535 && V > 0, "argmax_advance: M=%d V=%d", M, V);
    MXH_REQUIRE(ws_bytes >= argmax_ws_bytes(M, V), "argmax_advance: workspace of %zu bytes, %zu needed", ws_bytes,
                argmax_ws_bytes(M, V));
    MXH_REQUIRE(((uintptr_t)ws & 255) == 0, "argmax_advance: workspace must be 256-byte aligned");
    const int P = (V + kArgSlice - 1) / kArgSlice;
    const int64_t head = ((int64_t)(M + 1) * 4 + 255) / 256 * 256;
    uint8_t* w = static_cast<uint8_t*>(ws);
    ArgWs a{reinterpret_cast<uint32_t*>(w), reinterpret_cast<float*>(w + head),
            reinterpret_cast<int32_t*>(w + head + (int64_t)M * P * 4)};
    hipLaunchKernelGGL(argmax_kernel, dim3(P, M), dim3(256), 0, mxh::as_stream(stream), logits, V, M, ids, dpos, a);
    return mxh::launch_status("argmax_advance");
}
