"""CPU restatement of the reference's decode attention and KV write -- test
infrastructure (only tests/ use it).

Reference:
  f32_to_e4m3    src/ext/mxfp4_decode.cu:437-455   (KV byte encoder)
  e4m3_to_f32    src/ext/mxfp4_decode.cu:355-364   (KV byte decoder)
  kv_write       src/ext/mxfp4_decode.cu:457-489, binding mxfp4_decode_binding.cpp:161-173
  attn_decode    src/ext/mxfp4_decode.cu:366-430, binding mxfp4_decode_binding.cpp:213-230

The byte codec is the reference's own, not OCP E4M3: the encoder rounds the
3-bit mantissa half away from zero (lroundf), maps magnitudes below 2^-6 to
codes 0 / 1 (lroundf(a * 64)) and saturates everything that rounds to
exponent field 15 to 0x7F; the decoder reads subnormal codes as m * 2^-6 and
exponent-15 codes as 448 * (1 + m/8).  tests/test_oracle_attn.py pins both
against torch's OCP float8_e4m3fn where the two definitions agree and against
closed forms where they do not.

The reference's batch step writes its cache with torch instead
(runtime/model_runner_v2.py:256-257, k.to(torch.float8_e4m3fn)), read back by
the same attn_decode: e4m3_torch_encode restates that conversion (round to
nearest even, 0x7F above 464 and for inf/NaN); tests/test_oracle_attn.py pins
it against torch on every bf16 bit pattern.
"""
import numpy as np


def e4m3_ref_encode(v):
    """float32 array -> uint8 codes, the reference's f32_to_e4m3."""
    v = np.asarray(v, np.float32)
    sign = np.where(v < 0, 0x80, 0).astype(np.uint8)
    a = np.abs(v).astype(np.float32)
    f, e = np.frexp(a)                                  # a = f * 2^e, f in [0.5, 1)
    eb = e.astype(np.int64) + 6
    man = (a / np.ldexp(np.float32(1.0), e - 1)).astype(np.float32)
    x = ((man - np.float32(1.0)) * np.float32(8.0)).astype(np.float64)
    q = np.floor(x + 0.5).astype(np.int64)              # lroundf of a non-negative value
    carry = q == 8
    q = np.where(carry, 0, q)
    eb = np.where(carry, eb + 1, eb)
    sub = np.floor(np.minimum(a.astype(np.float64) * 64.0, 64.0) + 0.5).astype(np.int64).clip(0, 7)
    sat = eb >= 15
    eb = np.where(sat, 15, eb)
    q = np.where(sat, 7, q)
    normal = (sign.astype(np.int64) | ((eb & 15) << 3) | (q & 7)).astype(np.uint8)
    out = np.where(eb <= 0, (sign.astype(np.int64) | sub).astype(np.uint8), normal)
    return np.where(a == 0, sign, out).astype(np.uint8)


def e4m3_torch_encode(v):
    """float32 array -> uint8 codes of torch's float -> float8_e4m3fn: the
    nearest E4M3 value, ties to the even mantissa; subnormals q * 2^-9 below
    2^-6; magnitudes above 464 (which round past the largest finite 448),
    inf and NaN -> 0x7F; the sign bit is the input's."""
    v = np.asarray(v, np.float32)
    sign = ((v.view(np.uint32) >> 24) & 0x80).astype(np.int64)
    a = np.abs(v).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        f, e = np.frexp(np.where(np.isfinite(a), a, 1.0))      # a = f * 2^e, f in [0.5, 1)
        q = np.rint((2.0 * f - 1.0) * 8.0).astype(np.int64)    # mantissa of 2f in [1, 2)
        eb = e.astype(np.int64) - 1 + 7
        carry = q == 8
        q = np.where(carry, 0, q)
        eb = np.where(carry, eb + 1, eb)
        normal = (eb << 3) | q
        sub = np.rint(np.where(np.isfinite(a), a, 0.0) * 512.0).astype(np.int64)
        code = np.where(a < 2.0 ** -6, sub, normal)
        code = np.where(~(a <= 464.0), 0x7F, code)
    return (sign | code).astype(np.uint8)


def e4m3_ref_decode(b):
    """uint8 codes -> float32, the reference's e4m3_to_f32."""
    b = np.asarray(b, np.uint8).astype(np.int64)
    e = (b >> 3) & 15
    m = b & 7
    normal = (1.0 + m / 8.0) * np.exp2(e - 7.0)
    v = np.where(e == 0, m * 2.0 ** -6, np.where(e == 15, 448.0 * (1.0 + m / 8.0), normal))
    return np.where(b & 0x80, -v, v).astype(np.float32)


def kv_write_ref(k, v, kvk, kvv, base, codec=0):
    """k, v (M, Hkv, D) float32 (bf16 values); writes rows base+m < max_pos of
    the uint8 caches (max_pos, Hkv, D) in place; base < 0 writes nothing.
    codec 0: the decode extension's kv_write encoder; 1: torch's."""
    enc = e4m3_torch_encode if codec else e4m3_ref_encode
    kvk, kvv = np.asarray(kvk), np.asarray(kvv)
    M = k.shape[0]
    if base < 0:
        return kvk, kvv
    for m in range(M):
        pos = base + m
        if pos < kvk.shape[0]:
            kvk[pos] = enc(k[m])
            kvv[pos] = enc(v[m])
    return kvk, kvv


def attn_decode_ref(q, kvk, kvv, base):
    """q (M, Hq, D) float32 (bf16 values), caches (max_pos, Hkv, D) uint8.
    Token m at pos = base + m attends to positions 0..pos of its kv head
    h // (Hq/Hkv): raw scores q . k, softmax of score * fp32(1/sqrt(D)),
    weighted sum of v; float64.  Returns (o (M, Hq, D), scores list of
    (Hq, S_m) arrays); rows with pos outside [0, max_pos) are None."""
    M, Hq, D = q.shape
    max_pos, Hkv, _ = kvk.shape
    G = Hq // Hkv
    inv = np.float64(np.float32(1.0) / np.sqrt(np.float32(D)))
    kd = e4m3_ref_decode(kvk).astype(np.float64)
    vd = e4m3_ref_decode(kvv).astype(np.float64)
    o = np.full((M, Hq, D), np.nan)
    scores = []
    for m in range(M):
        pos = base + m
        if pos < 0 or pos >= max_pos:
            scores.append(None)
            continue
        S = pos + 1
        sm = np.zeros((Hq, S))
        for h in range(Hq):
            g = h // G
            s = kd[:S, g, :] @ q[m, h].astype(np.float64)
            sm[h] = s
            x = s * inv
            p = np.exp(x - x.max())
            o[m, h] = (p @ vd[:S, g, :]) / p.sum()
        scores.append(sm)
    return o, scores
