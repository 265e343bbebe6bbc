// mx_device.h -- gfx950 device primitives for the MXFP4 MoE path.
//
// * Bit-exact MXFP4 quantizer (contract: quant/fp4_format.py:21-148).
//   E8M0: smallest 2^e with amax <= 6*2^e, clamp [-127,127], 0 -> 127, decided
//   from the fp32 exponent/mantissa fields.  This equals the reference's
//   frexp(amax/6) for every normal amax and also covers amax/6 underflow,
//   where src/ext/mxfp4_common.cuh:42-50 would return 127.
//   E2M1: nearest magnitude, ties toward the larger one, sign = (x < 0).
//   The hardware converts (v_cvt_scalef32_pk_fp4_*) round ties to even and are
//   therefore NOT used for the bit-exact path.
// * CDNA4 block-scaled MFMA wrappers (v_mfma_scale_f32_{16x16x128,32x32x64}_f8f6f4).
//   Operand layouts, measured on MI355X with a random-input probe:
//     16x16x128, FP4 A and B: lane l holds row (A) / column (B) l%16 and the
//       32 K-values 32*(l/16) .. +31 of the 128-K chunk as 16 bytes, nibble t
//       of the chunk at byte t/2 (low nibble first); the lane's own E8M0 scale
//       (byte 0 of the scale VGPR with op_sel 0) covers exactly those 32 values.
//     16x16x128, FP8 (E4M3) A: lane l holds row l%16, bytes 0..15 = K
//       16g..16g+15 and bytes 16..31 = K 64+16g..64+16g+15 (g = l/16); the
//       scale of row r, 32-block b is read from lane r+16b.
//     16x16 accumulator: lane l, element i = D[4*(l/16)+i][l%16].
//     32x32x64, FP4: lane l holds row/column l%32, K 32*(l/32)..+31;
//       accumulator element i of lane l = D[8*(i/4)+4*(l/32)+i%4][l%32].
//   Because A and B of the same lane pair always cover the same K set, any
//   permutation of whole 32-element blocks applied to both operands leaves the
//   product unchanged; the kernels use that freedom to give each lane
//   contiguous memory.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int kBlock = 32;

// ---------------------------------------------------------------- quantizer
// E8M0 code of the smallest 2^e with amax <= 6*2^e (quant/fp4_format.py:73-88).
// amax <= 0 gives 127 (:78-79); so does an infinite amax, because the
// reference's frexp(inf) yields exponent 0 (:81-88).
__device__ __forceinline__ uint32_t e8m0_code(float amax) {
    if (!(amax > 0.0f) || !(amax <= 3.402823466e38f)) return 127u;
    uint32_t bits = __float_as_uint(amax);
    int ex = (int)(bits >> 23);
    uint32_t frac = bits & 0x7FFFFFu;
    int x;
    if (ex == 0) {  // denormal amax: renormalise
        int p = 31 - __clz((int)frac);
        x = p - 149;
        frac = (frac << (23 - p)) & 0x7FFFFFu;
    } else {
        x = ex - 127;
    }
    // amax = (1+f)*2^x <= 1.5*2^(e+2)  <=>  e = x-2 if (1+f) <= 1.5 else x-1
    int e = (frac <= 0x400000u) ? x - 2 : x - 1;
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
    return (uint32_t)(e + 127);
}

// 2^(127-code) as fp32: the reciprocal of the block scale.  Exact; for finite
// amax the code never exceeds 253 so the result is a normal number.
__device__ __forceinline__ float e8m0_inv_scale(uint32_t code) {
    return code < 254u ? __uint_as_float((254u - code) << 23) : __uint_as_float(0x00400000u >> (code - 254u));
}

// E2M1 code of x = v / scale: nearest magnitude, ties up, clamp at 6,
// sign bit from (x < 0) (quant/fp4_format.py:24-46).  The magnitude code is
// the count of the thresholds 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5 that |x|
// reaches.  From 1 up the E2M1 grid is a float with one mantissa bit, so
// there the count is |x| rounded half-up to one mantissa bit (add half an
// ulp of that grid, 2^21, to the fp32 bits and keep exponent + top mantissa
// bit) minus the code offset, clamped to [2, 7]; below 1 it is the first two
// comparisons.  Equal to the plain threshold count on all 2^32 inputs (NaN
// -> 0, -0 -> 0), in about half the instructions.
__device__ __forceinline__ uint32_t e2m1_code(float x) {
    const float a = __builtin_fabsf(x);
    const int hi = min(max((int)((__float_as_uint(a) + 0x200000u) >> 22) - 252, 2), 7);
    const uint32_t lo = (uint32_t)(a >= 0.25f) + (uint32_t)(a >= 0.75f);
    const uint32_t m = a >= 1.0f ? (uint32_t)hi : lo;
    return m | (x < 0.0f ? 8u : 0u);
}

// Quantize 8 consecutive values of a 32-block whose scale code is known:
// returns the 8 nibbles packed LSB-first into 32 bits.
__device__ __forceinline__ uint32_t e2m1_pack8(const float v[8], float inv) {
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) r |= e2m1_code(v[i] * inv) << (4 * i);
    return r;
}

// The same codes from the hardware conversion, for x = v * inv with v exact
// in fp16 or bf16 (at most 11 significant bits) and inv a power of two.
// v_cvt_scalef32_pk_fp4_f32 rounds to nearest even and saturates at 6, gives
// -0 the code 8 and NaN the code 7 or 15; e2m1_code rounds ties up and gives
// +-0 and NaN the code 0.  Moving x one fp32 ulp away from zero turns every
// tie into a value above it, and with at most 11 significant bits no value
// below a tie reaches it; zero and NaN become +0, infinities stay (6).  Equal
// to e2m1_code on every bf16 and every fp16 bit pattern (checked on the GPU
// for all 2^17).  Fewer than half the instructions of e2m1_code.
__device__ __forceinline__ float e2m1_hw_arg(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t bump = (b & 0x7F800000u) != 0x7F800000u ? 1u : 0u;
    return __builtin_fabsf(x) > 0.0f ? __uint_as_float(b + bump) : 0.0f;
}
// Two codes, x0 in the low nibble of byte `sel` of `old`, x1 in the high one.
template <int SEL>
__device__ __forceinline__ uint32_t e2m1_hw_pair(uint32_t old, float x0, float x1) {
    return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(old, e2m1_hw_arg(x0), e2m1_hw_arg(x1), 1.0f, SEL);
}
// e2m1_pack8 for values exact in fp16 or bf16 (see e2m1_hw_arg).
__device__ __forceinline__ uint32_t e2m1_pack8_short(const float v[8], float inv) {
    uint32_t r = 0;
    r = e2m1_hw_pair<0>(r, v[0] * inv, v[1] * inv);
    r = e2m1_hw_pair<1>(r, v[2] * inv, v[3] * inv);
    r = e2m1_hw_pair<2>(r, v[4] * inv, v[5] * inv);
    r = e2m1_hw_pair<3>(r, v[6] * inv, v[7] * inv);
    return r;
}

// ---------------------------------------------------------------- scale loads
// MFMA K-steps st0 .. st0+3 of a lane in group q (block 4*st + q at step st)
// need the scale bytes 4*(st0 + j) + q, j < 4, of one row: bytes [4*st0,
// 4*st0 + 16) of the row hold them all, so when that span lies inside the
// row and the row address is 8-byte aligned, two 8-byte loads replace the
// four byte loads (byte j of the lane is then byte q of dword j); otherwise
// the lane loads its four bytes (addresses clamped into the row).
//
// The loads only fill registers: the byte is picked at use (seg_scale_at).
// A load result consumed while a segment is still being issued makes the
// compiler wait for every load in flight there, which turns the prefetch of
// a segment into one memory round trip per segment.
struct SegScales {
    uint32_t d[4];
    bool words;   // d holds dwords (pick byte q) rather than the lane's bytes
};

__device__ __forceinline__ void seg_scales_issue(SegScales& r, const uint8_t* srow, int q, int st0, int nch) {
    const uint8_t* p = srow + 4 * st0;
    r.words = 4 * st0 + 16 <= nch && (reinterpret_cast<uintptr_t>(p) & 7) == 0;
    if (r.words) {
        const uint2 v0 = *reinterpret_cast<const uint2*>(p), v1 = *reinterpret_cast<const uint2*>(p + 8);
        r.d[0] = v0.x; r.d[1] = v0.y; r.d[2] = v1.x; r.d[3] = v1.y;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) r.d[j] = srow[min(4 * (st0 + j) + q, nch - 1)];
    }
}

// The scale code of step st0 + j; out-of-range steps or blocks, and !ok,
// give code 127 (scale 1, zero data).
__device__ __forceinline__ uint32_t seg_scale_at(const SegScales& r, int j, bool ok, int q, int st0, int steps,
                                                 int nch) {
    const uint32_t v = r.words ? (r.d[j] >> (8 * q)) & 0xFFu : r.d[j];
    return (ok && st0 + j < steps && 4 * (st0 + j) + q < nch) ? v : 127u;
}


// ---------------------------------------------------------------- FP4 decode
// E2M1 nibble -> fp32 (used by reference-style epilogues and tests only).
__device__ __forceinline__ float e2m1_value(uint32_t c) {
    const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
    float v = mag[c & 7u];
    return (c & 8u) ? -v : v;
}

// ---------------------------------------------------------------- MFMA
__device__ __forceinline__ v4f mfma16_fp4(uint4 a, uint4 b, v4f c, uint32_t sa, uint32_t sb) {
    v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    v8i bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 4, 4, 0, (int)sa, 0, (int)sb);
}

// A = E4M3 (32 bytes per lane), B = FP4.
__device__ __forceinline__ v4f mfma16_fp8a_fp4b(v8i a, uint4 b, v4f c, uint32_t sa, uint32_t sb) {
    v8i bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bv, c, 0, 4, 0, (int)sa, 0, (int)sb);
}

__device__ __forceinline__ v16f mfma32_fp4(uint4 a, uint4 b, v16f c, uint32_t sa, uint32_t sb) {
    v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    v8i bv = {(int)b.x, (int)b.y, (int)b.z, (int)b.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 4, 4, 0, (int)sa, 0, (int)sb);
}

// Materialises an MFMA result at this point of wave-uniform control flow.
// An MFMA reads the operands of all 64 lanes, but the compiler models it as a
// per-lane operation: when only some lanes consume the result (`if (lane <
// 16) store(acc)`), it may sink the MFMA chain -- and the per-lane selects
// that build its operands -- into that branch, where the operands of the other
// lanes are never written.  The empty volatile asm uses and redefines the
// value, so the chain must complete before any lane-dependent branch.
__device__ __forceinline__ void pin(v4f& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(v16f& v) { asm volatile("" : "+v"(v)); }
// The same for accumulators kept in AGPRs (one wave per SIMD, 256 AGPRs of
// accumulators): pinning them to VGPRs would force copies through the loop.
__device__ __forceinline__ void pin_acc(v16f& v) { asm volatile("" : "+a"(v)); }

// ---------------------------------------------------------------- misc
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// fp32 -> nearest fp16 (RNE, overflow to inf) -> fp32: the rounding torch's
// .to(torch.half) applies.
__device__ __forceinline__ float round_to_f16(float f) { return (float)(_Float16)f; }

// fp32 -> bf16 bits, round to nearest even (finite inputs).
// Two fp32 -> bf16 (RNE, as f32_to_bf16_rne for every non-NaN input) in one
// v_cvt_pk_bf16_f32: a in the low half, b in the high half.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// h is a rounded fp32 value, as in the reference: no contraction of its last
// product into whatever the caller computes from it next (an FMA there would
// make the result depend on the surrounding code).
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
    // h = g / (1 + exp(-g)) * u, fp32 (src/ext/mxfp4_decode.cu:258)
    return (g / (1.0f + expf(-g))) * u;
}

// silu_mul on the hardware exp2 and reciprocal (a few ulp from silu_mul):
// for the fused decode kernels, whose h is split into three E4M3 terms (a
// resolution of 2^-13.8 of the block amax), and the prefill MoE, whose h is rounded to
// fp16 and then to 4-bit codes, which a few-ulp change moves only for an h
// within ~1e-6 (relative) of a rounding threshold.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);   // exp(-g); +inf for g < -88
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Lane exchanges by DPP (a VALU operand modifier, no LDS round trip; a
// shuffle through ds_bpermute costs an LDS-path latency per step).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppQuadNext1 = 0xF9;       // quad_perm [1,2,3,3]: lane q*4 reads q*4+1
constexpr int kDppQuadNext2 = 0xEE;       // quad_perm [2,3,2,3]: lane q*4 reads q*4+2
constexpr int kDppRowHalfMirror = 0x141;  // lane i of 8 reads 7 - i
constexpr int kDppRowMirror = 0x140;      // lane i of 16 reads 15 - i

// The wave's sum by the butterfly xor 32, 16, 8, 4, 2, 1 (each lane adds
// its partner's partial sum), in every lane: the bits of
//     for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
// with the lane exchanges kept in the VALU -- the gfx950 permlane swaps for
// xor 32 and 16 (lanes of VDST's upper half / odd rows trade with VSRC's
// lower half / even rows), a row rotation by 8, quad xor 3 then the half-row
// mirror (lane i of 8 reads (7 - i) ^ 3 = i ^ 4), quad xor 2 and 1 -- instead
// of six shuffles through the LDS path.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
    const int lane = threadIdx.x & 63;
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v += __uint_as_float(lane < 32 ? r[1] : r[0]);
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v += __uint_as_float(((lane >> 4) & 1) ? r[0] : r[1]);
    }
    v += dpp<0x128>(v);                             // row_ror 8: lane i of 16 reads i ^ 8
    v += dpp<kDppRowHalfMirror>(dpp<0x1B>(v));      // quad_perm [3,2,1,0], then the half-row mirror
    v += dpp<kDppQuadXor2>(v);
    v += dpp<kDppQuadXor1>(v);
    return v;
}

// Reduction over each row of 16 lanes, the row's total in every lane of it.
// Quad xor 1, quad xor 2, half-row mirror, row mirror: after the quad steps
// every lane of a quad holds the same value, so the mirrors pair each quad
// (half-row) with the same other one as xor 4 (xor 8) would, and the result
// has the bits of the xor-1,2,4,8 butterfly (the operations are commutative).
template <bool MAX>
__device__ __forceinline__ float row16_reduce(float v) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    v = op(v, dpp<kDppQuadXor1>(v));
    v = op(v, dpp<kDppQuadXor2>(v));
    v = op(v, dpp<kDppRowHalfMirror>(v));
    return op(v, dpp<kDppRowMirror>(v));
}

// Reduction over the wave, result in every lane: the row reduction above,
// then the four row results ((r0 op r1) op (r2 op r3)).  For the maximum,
// NaN inputs are ignored (maxNum), so NaN can mark "no value".
template <bool MAX>
__device__ __forceinline__ float wave_reduce_dpp(float v) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    v = row16_reduce<MAX>(v);
    return op(op(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))),
              op(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48))));
}

// Router top-k of one row by one wave (runtime/model_runner_v2.py:189-192:
// softmax, top-k, renormalise).  The softmax is monotonic, so the k winners
// are taken in descending logit order (k rounds of a wave maximum; exact
// ties: lower index), which is torch.topk's order on the probabilities except
// where two different logits round to the same probability (an order torch
// leaves unspecified).  Weights: e_r = exp(l_r - l_max) of the winners;
// renormalised w_r = e_r / sum_r e_r (rank order), which is
// topv_r / sum(topv) of the probabilities; otherwise w_r = e_r / sum over
// the row.  Lane r < k receives rank r.  The row has n <= 64*NPL entries,
// element i*64 + lane held by the lane; k <= 64.  NaN logits are never
// chosen.
// wave_topk_regs takes the row from registers: lv[i] = element i*64 + lane
// (any value for i*64 + lane >= n).
template <int NPL>
__device__ __forceinline__ void wave_topk_regs(const float (&lv)[NPL], int n, int k, int norm, int& id, float& w) {
    const int lane = threadIdx.x & 63;
    const float kNone = __builtin_nanf("");
    float v[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) v[i] = i * 64 + lane < n ? lv[i] : kNone;
    float my_l = 0.0f;
    int my_i = 0;
    for (int r = 0; r < k; ++r) {
        float b = v[0];
#pragma unroll
        for (int i = 1; i < NPL; ++i) b = fmaxf(b, v[i]);
        const float m = wave_reduce_dpp<true>(b);
        int win = 0;
#pragma unroll
        for (int i = NPL - 1; i >= 0; --i) {   // the lowest index holding m wins
            const uint64_t bal = __ballot(v[i] == m);
            if (bal) win = i * 64 + (int)__builtin_ctzll(bal);
        }
        if (lane == r) {
            my_l = m;
            my_i = win;
        }
        if ((win & 63) == lane) {
#pragma unroll
            for (int i = 0; i < NPL; ++i)
                if (i == (win >> 6)) v[i] = kNone;
        }
    }
    const float lmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_l), 0));
    const float e = lane < k ? expf(my_l - lmax) : 0.0f;
    float den = 0.0f;
    if (norm) {
        for (int r = 0; r < k; ++r) den += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), r));
    } else {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < NPL; ++i)
            if (i * 64 + lane < n) s += expf(lv[i] - lmax);
        den = wave_reduce_dpp<false>(s);
    }
    id = my_i;
    w = e / den;
}

template <int NPL>
__device__ __forceinline__ void wave_topk(const float* __restrict__ lg, int n, int k, int norm, int& id, float& w) {
    const int lane = threadIdx.x & 63;
    float lv[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int idx = i * 64 + lane;
        lv[i] = idx < n ? lg[idx] : 0.0f;
    }
    wave_topk_regs<NPL>(lv, n, k, norm, id, w);
}

}  // namespace mx
