/* mxfp4_oracle.c -- C restatement of the MXFP4 quantizer (test infrastructure).
 *
 * Test-only checker, never shipped and never called by the product path.  A
 * second, independently written implementation of the bit-exact contract of
 * quant/fp4_format.py (E2M1 ties-to-larger-magnitude, smallest-power-of-two
 * E8M0 scale, LSB-first packing) and of the row quantizer / layout of
 * quant/quantize_mxfp4.py:110-160.  The numpy restatement (oracle/mxfp4.py)
 * decides the scale from frexp in float64; this one decides it from the fp32
 * exponent and mantissa fields, and encodes E2M1 with threshold compares
 * rather than a sorted search, so the two can be swept against each other.
 *
 * Build: see oracle/Makefile (gcc -O2 -shared -fPIC).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Smallest e with amax <= 6 * 2^e, clamped to [-127, 127]; code e + 127;
 * amax <= 0 -> 127.  quant/fp4_format.py:73-88. */
uint8_t mxo_e8m0_code(float amax) {
    if (!(amax > 0.0f) || isinf(amax)) return 127; /* frexp(inf) -> exponent 0 */
    uint32_t bits;
    memcpy(&bits, &amax, 4);
    int32_t ex = (int32_t)((bits >> 23) & 0xFF);
    uint32_t frac = bits & 0x7FFFFF;
    int32_t x; /* amax = (1 + frac/2^23) * 2^x */
    if (ex == 0) { /* denormal: renormalise */
        int p = 31 - __builtin_clz(frac);          /* msb index, 0..22 */
        x = p - 149;
        frac = (frac << (23 - p)) & 0x7FFFFF;
    } else {
        x = ex - 127;
    }
    /* (1+f) * 2^x <= 1.5 * 2^(e+2)  <=>  e = x-2 when (1+f) <= 1.5, else x-1 */
    int32_t e = (frac <= 0x400000u) ? x - 2 : x - 1;
    if (e < -127) e = -127;
    if (e > 127) e = 127;
    return (uint8_t)(e + 127);
}

/* The reference's own formula (quant/fp4_format.py:78-88): frexp of amax/6 in
 * double, m == 0.5 meaning an exact power of two.  Kept only to sweep against
 * mxo_e8m0_code. */
uint8_t mxo_e8m0_code_frexp(float amax) {
    if (!(amax > 0.0f)) return 127;
    if (isinf(amax)) return 127;
    int e;
    double m = frexp((double)amax / 6.0, &e);
    int ep = (m == 0.5) ? e - 1 : e;
    if (ep < -127) ep = -127;
    if (ep > 127) ep = 127;
    return (uint8_t)(ep + 127);
}

/* E2M1 code of x (already divided by the block scale): nearest magnitude with
 * ties to the larger one, clamp at 6, sign bit = (x < 0). */
uint8_t mxo_e2m1_code(float x) {
    float a = fabsf(x);
    uint8_t m;
    if (a < 0.25f) m = 0;
    else if (a < 0.75f) m = 1;
    else if (a < 1.25f) m = 2;
    else if (a < 1.75f) m = 3;
    else if (a < 2.5f) m = 4;
    else if (a < 3.5f) m = 5;
    else if (a < 5.0f) m = 6;
    else m = 7;
    return (uint8_t)(m | ((x < 0.0f) ? 8 : 0));
}

/* 2^(code - 127) as fp32 (2^-127 is a denormal). */
float mxo_scale(uint8_t code) { return ldexpf(1.0f, (int)code - 127); }

/* Rows (n, k) fp32 -> packed (n, kp/2) + scale codes (n, kp/32); rows are
 * zero-padded to kp (a multiple of 32, >= k). */
void mxo_quantize_rows(const float* w, int64_t n, int64_t k, int64_t kp,
                       uint8_t* packed, uint8_t* scales) {
    for (int64_t r = 0; r < n; ++r) {
        const float* row = w + r * k;
        for (int64_t b = 0; b < kp / 32; ++b) {
            float v[32];
            float amax = 0.0f;
            for (int t = 0; t < 32; ++t) {
                int64_t c = b * 32 + t;
                v[t] = (c < k) ? row[c] : 0.0f;
                float a = fabsf(v[t]);
                if (a > amax) amax = a;
            }
            uint8_t sc = mxo_e8m0_code(amax);
            scales[r * (kp / 32) + b] = sc;
            float s = mxo_scale(sc);
            for (int t = 0; t < 32; t += 2) {
                uint8_t lo = mxo_e2m1_code(v[t] / s);
                uint8_t hi = mxo_e2m1_code(v[t + 1] / s);
                packed[r * (kp / 2) + b * 16 + t / 2] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

/* Exhaustive sweep of every positive finite fp32 amax in [lo_bits, hi_bits):
 * counts disagreements between the field-based and the frexp-based scale
 * rules, and verifies 3 < amax/2^e <= 6 wherever e is unclamped.  Returns the
 * number of violations; the first offending bit pattern goes to *first. */
int64_t mxo_sweep_scale(uint32_t lo_bits, uint32_t hi_bits, uint32_t* first) {
    int64_t bad = 0;
    for (uint32_t b = lo_bits; b < hi_bits; ++b) {
        float a;
        memcpy(&a, &b, 4);
        uint8_t c1 = mxo_e8m0_code(a), c2 = mxo_e8m0_code_frexp(a);
        int ok = (c1 == c2);
        int e = (int)c1 - 127;
        if (ok && e > -127 && e < 127) {
            double r = ldexp((double)a, -e);
            ok = (r > 3.0 && r <= 6.0);
        }
        if (!ok) {
            if (bad == 0 && first) *first = b;
            ++bad;
        }
    }
    return bad;
}
