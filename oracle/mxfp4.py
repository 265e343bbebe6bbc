"""MXFP4 format restatement (numpy) -- test infrastructure only, never shipped.

Restates the reference's bit-exact contract:

* E2M1 element codec       quant/fp4_format.py:21-53
* E8M0 block-scale rule    quant/fp4_format.py:59-88
* LSB-first nibble packing quant/fp4_format.py:126-148
* row quantizer / layout   quant/quantize_mxfp4.py:110-160 (MXFP4_BLOCK = 32,
                           zero padding of K to Kp = ceil(K/32)*32, row-major
                           packed (n, Kp/2) u8 + scale codes (n, Kp/32) u8)
* dequant                  runtime/weight_store.py:27-65

Where the reference's numpy weight packer (quant/quantize_mxfp4.py:135-141)
and quant/fp4_format.py disagree -- fp32 amax within ~2 ulps above 6*2^k, and
amax <= ~6e-30 -- this restatement follows quant/fp4_format.py, which is the
stated contract.  The two agree for every bf16-origin block with amax > 6e-30.

The scale rule is written here as an exact integer decision on the frexp
decomposition of amax, not as the reference's frexp(amax/6): with
amax = m * 2^q (m in [0.5, 1)), amax <= 6 * 2^e holds for e = q-3 exactly when
m <= 0.75, otherwise the smallest e is q-2.
"""
import numpy as np

BLOCK = 32                      # quant/quantize_mxfp4.py:35 (MXFP4_BLOCK)
E8M0_BIAS = 127                 # quant/fp4_format.py:59
# E2M1 magnitudes, quant/fp4_format.py:21
E2M1_MAG = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
# Midpoints between neighbouring magnitudes; a value equal to a midpoint takes
# the larger magnitude (quant/fp4_format.py:39, "tie -> upper").
E2M1_MIDPOINTS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float64)


def e2m1_encode(x):
    """Nearest E2M1 code, ties toward the larger magnitude, clamp at 6.

    Sign bit (bit 3) is ``x < 0`` evaluated on x itself, so -0.0 gives code 0
    and tiny negatives that round to magnitude 0 give code 8.
    quant/fp4_format.py:24-46.
    """
    xa = np.asarray(x)
    a = np.abs(xa.astype(np.float64))
    mag = np.searchsorted(E2M1_MIDPOINTS, a, side="right").astype(np.uint8)
    sign = (xa.astype(np.float64) < 0).astype(np.uint8)
    return ((sign << 3) | mag).astype(np.uint8)


def e2m1_decode(codes):
    """Code -> float32 value, quant/fp4_format.py:49-53."""
    c = np.asarray(codes).astype(np.uint8) & 0xF
    v = E2M1_MAG[c & 7]
    return np.where((c >> 3) != 0, -v, v).astype(np.float32)


def e8m0_code(amax):
    """Block amax -> E8M0 code of the smallest 2^e with amax <= 6 * 2^e.

    e is clamped to [-127, 127]; amax <= 0 gives 127 (scale 1.0).  An infinite
    amax also gives 127: the reference computes frexp(inf) = (inf, 0), i.e.
    exponent 0.  quant/fp4_format.py:73-88.  Vectorised; amax is any float array.
    """
    a = np.asarray(amax, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        m, q = np.frexp(np.where(np.isfinite(a), a, 1.0))
    e = np.where(m <= 0.75, q - 3, q - 2)
    e = np.clip(e, -E8M0_BIAS, E8M0_BIAS)
    return np.where((a > 0) & np.isfinite(a), e + E8M0_BIAS, E8M0_BIAS).astype(np.uint8)


def e8m0_scale_f32(codes):
    """E8M0 code -> float32 scale 2^(code-127) (2^-127 is an fp32 denormal,
    2^127 is finite).  quant/fp4_format.py:69-70."""
    c = np.asarray(codes).astype(np.int64)
    return np.ldexp(np.float32(1.0), (c - E8M0_BIAS).astype(np.int32)).astype(np.float32)


def pack_nibbles(codes):
    """LSB-first: byte j = c[2j] | c[2j+1] << 4; an odd tail is padded with 0.
    Returns (packed u8, pad).  quant/fp4_format.py:126-137."""
    c = np.asarray(codes, dtype=np.uint8).reshape(-1)
    pad = c.size % 2
    if pad:
        c = np.concatenate([c, np.zeros(1, np.uint8)])
    return (c[0::2] | (c[1::2] << 4)).astype(np.uint8), pad


def unpack_nibbles(packed, n=None):
    """Inverse of pack_nibbles, quant/fp4_format.py:140-148."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    out = np.empty(p.size * 2, np.uint8)
    out[0::2] = p & 0xF
    out[1::2] = p >> 4
    return out if n is None else out[:n]


def padded_k(k):
    return (k + BLOCK - 1) // BLOCK * BLOCK


def quantize_rows(w, kp=None):
    """fp32 rows (n, k) -> (packed (n, Kp/2) u8, scale codes (n, Kp/32) u8).

    Restates quant/quantize_mxfp4.py:110-160: rows zero-padded along K to Kp
    (:124-128); per 32-block amax -> E8M0 code (scale rule of
    quant/fp4_format.py:73-88); elements divided by the fp32 scale (exact
    power-of-two division, :145) and E2M1-encoded (:146); packed row-major
    LSB-first (:147).  ``kp`` may exceed ceil32(k) to pad further (used for
    activations quantized against a weight's Kp).
    """
    w = np.ascontiguousarray(np.asarray(w, dtype=np.float32))
    if w.ndim == 1:
        w = w[None, :]
    n, k = w.shape
    kp = padded_k(k) if kp is None else int(kp)
    assert kp % BLOCK == 0 and kp >= k
    wf = np.zeros((n, kp), np.float32)
    wf[:, :k] = w
    blocks = wf.reshape(n, kp // BLOCK, BLOCK)
    amax = np.max(np.abs(blocks), axis=-1)
    codes_s = e8m0_code(amax)
    scale = e8m0_scale_f32(codes_s)
    with np.errstate(under="ignore"):
        scaled = (blocks / scale[..., None]).astype(np.float32)
    codes = e2m1_encode(scaled).reshape(n, kp)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    return packed, codes_s


def dequant_rows(packed, scales, k=None):
    """(n, Kp/2) u8 + (n, Kp/32) u8 -> fp32 (n, k); value = sign * table *
    2^(s-127), exact in fp32.  runtime/weight_store.py:27-44."""
    p = np.asarray(packed, dtype=np.uint8)
    s = np.asarray(scales, dtype=np.uint8)
    n = p.shape[0]
    kp = p.shape[1] * 2
    codes = np.empty((n, kp), np.uint8)
    codes[:, 0::2] = p & 0xF
    codes[:, 1::2] = p >> 4
    vals = e2m1_decode(codes).reshape(n, kp // BLOCK, BLOCK).astype(np.float64)
    sc = np.ldexp(1.0, s.astype(np.int64) - E8M0_BIAS)
    out = (vals * sc[..., None]).reshape(n, kp).astype(np.float32)
    return out if k is None else out[:, :k]


def bf16_round(x):
    """fp32 -> nearest bf16 (round-to-nearest-even), returned as fp32 values.
    Matches torch's float->bfloat16 conversion for finite inputs."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def f16_round(x):
    """fp32 -> fp16 (RNE) -> fp32, the rounding the reference's `forward`
    applies to its activations (src/ext/mxfp4_binding.cpp:31)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
