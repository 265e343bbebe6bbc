"""Pins the CPU oracle's MXFP4 format (oracle/mxfp4.py, oracle/mxfp4_oracle.c).

Checks, in order of strength:
  * the reference's own self-test KATs (quant/fp4_format.py:154-198), as data
    in tests/golden/mxfp4_kat.json;
  * exhaustive sweeps over every bf16 bit pattern against a brute force in
    exact rational arithmetic (E2M1 nearest with ties to the larger magnitude;
    E8M0 smallest e with amax <= 6*2^e);
  * fp32 edge values around every 6*2^k and the whole denormal range, swept
    between the two independently written implementations (numpy frexp rule,
    C bit-field rule) and the reference's own frexp(amax/6) formula;
  * layout invariants of the row quantizer (row-major, LSB-first, zero
    padding) and dequant round trip / idempotence.
"""
import ctypes
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import cbuild
from oracle import mxfp4 as fmt

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TABLE = [Fraction(v) for v in (0, 0.5, 1, 1.5, 2, 3, 4, 6)]


def _kat():
    with open(os.path.join(GOLDEN, "mxfp4_kat.json")) as f:
        return json.load(f)


# ---------------------------------------------------------------- KATs
def test_reference_kat_decode_and_requantize():
    k = _kat()
    vals = fmt.e2m1_decode(np.array(k["decode_all"]["codes"], np.uint8))
    assert np.array_equal(vals, np.array(k["decode_all"]["values"], np.float32))
    rec = fmt.e2m1_encode(vals)
    assert rec.tolist() == k["requantize_all"]["expected"]


def test_reference_kat_points():
    k = _kat()
    for x, v in k["encode_points"]:
        assert float(fmt.e2m1_decode(fmt.e2m1_encode(np.float32(x)))) == v
    for c, v in k["decode_points"]:
        assert float(fmt.e2m1_decode(np.uint8(c))) == v
    for amax, scale in k["scale_points"]:
        code = int(fmt.e8m0_code(amax))
        assert float(fmt.e8m0_scale_f32(code)) == scale
        assert int(cbuild.lib().mxo_e8m0_code(amax)) == code
        assert amax / scale <= 6.0


def test_infinite_amax_gives_scale_one():
    # quant/fp4_format.py:81-88: math.frexp(inf) == (inf, 0) -> e = 0 -> code 127
    assert math.frexp(float("inf"))[1] == 0
    assert int(fmt.e8m0_code(np.float32(np.inf))) == 127
    assert int(cbuild.lib().mxo_e8m0_code(float("inf"))) == 127
    q, s = fmt.quantize_rows(np.array([[np.inf, -7.5, 1.0] + [0.0] * 29], np.float32))
    assert s[0, 0] == 127
    assert (q[0, 0] & 0xF) == 7 and (q[0, 0] >> 4) == 15 and (q[0, 1] & 0xF) == 2


def test_reference_kat_pack():
    k = _kat()["pack"]
    packed, pad = fmt.pack_nibbles(np.array(k["codes"], np.uint8))
    assert packed.tolist() == k["bytes"] and pad == k["pad"]
    assert fmt.unpack_nibbles(packed, n=len(k["codes"])).tolist() == k["codes"]


def test_reference_kat_linspace_chain():
    k = _kat()["linspace"]
    x = np.linspace(k["start"], k["stop"], k["num"], dtype=np.float32)
    q = fmt.e2m1_encode(x)
    p, _ = fmt.pack_nibbles(q)
    assert np.array_equal(fmt.unpack_nibbles(p, n=x.size), q)


# ---------------------------------------------------------------- exhaustive bf16
def _all_finite_bf16():
    bits = np.arange(1 << 16, dtype=np.uint32)
    f = fmt.bf16_bits_to_f32(bits)
    return f[np.isfinite(f)]


def _e2m1_bruteforce(x):
    """Exact nearest table magnitude, ties to the larger, clamp at 6."""
    a = abs(Fraction(float(x)))
    best = 0
    for i, t in enumerate(TABLE):
        d, db = abs(a - t), abs(a - TABLE[best])
        if d < db or d == db:  # later entries are larger: ties go up
            best = i
    return best | (8 if float(x) < 0 else 0)


def test_e2m1_exhaustive_bf16_vs_exact():
    # values in the quantizer's working range plus everything beyond 6
    x = _all_finite_bf16()
    x = x[np.abs(x) <= 16.0]
    got = fmt.e2m1_encode(x)
    want = np.array([_e2m1_bruteforce(v) for v in x], np.uint8)
    assert np.array_equal(got, want)
    # the C restatement (threshold compares) agrees as well
    L = cbuild.lib()
    sub = x[:: 7]
    assert [L.mxo_e2m1_code(float(v)) for v in sub] == [int(c) for c in fmt.e2m1_encode(sub)]


def _e8m0_exact(amax):
    """Smallest e with amax <= 6*2^e, clamped to [-127, 127], exact rationals."""
    a = Fraction(float(amax))
    if a <= 0:
        return 127
    e = math.frexp(float(amax))[1] - 3
    while a > 6 * Fraction(2) ** e:
        e += 1
    while a <= 6 * Fraction(2) ** (e - 1):
        e -= 1
    return max(-127, min(127, e)) + 127


def test_e8m0_exhaustive_bf16_vs_exact():
    x = _all_finite_bf16()
    x = np.unique(np.abs(x))
    got = fmt.e8m0_code(x)
    want = np.array([_e8m0_exact(v) for v in x], np.uint8)
    assert np.array_equal(got, want)
    L = cbuild.lib()
    assert [L.mxo_e8m0_code(float(v)) for v in x[::5]] == [int(c) for c in want[::5]]


def test_e8m0_fp32_edges_exact():
    """fp32 values within 3 ulps of 6*2^k for every k, plus denormals."""
    vals = []
    for k in range(-150, 126):
        c = np.float32(6.0 * 2.0 ** k)
        if c is None or not np.isfinite(c) or c == 0:
            continue
        v = c
        for _ in range(3):
            v = np.nextafter(v, np.float32(np.inf))
            vals.append(v)
        v = c
        for _ in range(3):
            v = np.nextafter(v, np.float32(0))
            vals.append(v)
        vals.append(c)
    vals += [np.float32(2.0 ** -149), np.float32(2.0 ** -148), np.float32(3 * 2.0 ** -149),
             np.finfo(np.float32).max]
    vals = np.array(vals, np.float32)
    got = fmt.e8m0_code(vals)
    want = np.array([_e8m0_exact(v) for v in vals], np.uint8)
    assert np.array_equal(got, want)
    L = cbuild.lib()
    assert [L.mxo_e8m0_code(float(v)) for v in vals] == want.tolist()


def test_c_sweep_against_reference_formula():
    """The C field rule equals frexp(amax/6) in double (the reference's own
    formula, quant/fp4_format.py:78-88) over the whole denormal range and
    +-2^12 ulps around every 6*2^k; the invariant 3 < amax/2^e <= 6 holds."""
    L = cbuild.lib()
    first = ctypes.c_uint32(0)
    assert L.mxo_sweep_scale(1, 1 << 23, ctypes.byref(first)) == 0, hex(first.value)
    for k in range(-147, 126):
        c = int(np.float32(6.0 * 2.0 ** k).view(np.uint32))
        lo, hi = max(1, c - 4096), min(0x7F800000, c + 4096)
        assert L.mxo_sweep_scale(lo, hi, ctypes.byref(first)) == 0, (k, hex(first.value))


# ---------------------------------------------------------------- rows / layout
def _rows(seed, n, k):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, k)).astype(np.float32)
    x *= np.power(2.0, rng.integers(-2, 3, size=(n, 1))).astype(np.float32)
    x[rng.random((n, k)) < 0.01] *= np.float32(8.0)
    return x


@pytest.mark.parametrize("n,k", [(96, 128), (128, 100), (7, 33), (3, 2048), (5, 1)])
def test_quantize_rows_numpy_vs_c(n, k):
    x = _rows(n * 1000 + k, n, k)
    q1, s1 = fmt.quantize_rows(x)
    q2, s2 = cbuild.quantize_rows_c(x)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    assert q1.shape == (n, fmt.padded_k(k) // 2) and s1.shape == (n, fmt.padded_k(k) // 32)


def test_quantize_rows_layout_is_row_major_lsb_first():
    # row r holds the value (r+1) at column c == r and zeros elsewhere
    n, k = 6, 64
    x = np.zeros((n, k), np.float32)
    for r in range(n):
        x[r, 2 * r + (r % 2)] = r + 1.0
    q, s = fmt.quantize_rows(x)
    for r in range(n):
        c = 2 * r + (r % 2)
        nib = (q[r, c // 2] >> (4 * (c % 2))) & 0xF
        assert nib == fmt.e2m1_encode(np.float32((r + 1.0) / float(fmt.e8m0_scale_f32(s[r, 0]))))
        others = q[r].copy()
        others[c // 2] &= np.uint8(0xF0 if c % 2 == 0 else 0x0F)
        assert not others.any()
        assert s[r, 1] == 127  # second block all zero -> code 127


def test_dequant_roundtrip_and_idempotence():
    x = _rows(7, 64, 256)
    q, s = fmt.quantize_rows(x)
    d = fmt.dequant_rows(q, s)
    # error at most half the spacing of the E2M1 grid times the block scale
    sc = fmt.e8m0_scale_f32(s).astype(np.float64)
    err = np.abs(d - x).reshape(64, 8, 32) / sc[..., None]
    assert err.max() <= 1.0 + 1e-6
    q2, s2 = fmt.quantize_rows(d)
    d2 = fmt.dequant_rows(q2, s2)
    assert np.array_equal(d, d2)  # dequantized grid values are fixed points
    # where the re-derived scale is unchanged the codes are too (-0 -> +0);
    # a block whose amax decoded to 3*2^e legitimately re-scales to 2^(e-1)
    codes = fmt.unpack_nibbles(q.reshape(-1)).reshape(64, 8, 32)
    codes2 = fmt.unpack_nibbles(q2.reshape(-1)).reshape(64, 8, 32)
    same = s == s2
    assert same.mean() > 0.5
    assert np.array_equal(np.where(codes == 8, 0, codes)[same], codes2[same])
    assert np.all(s2[~same] == s[~same] - 1)


def test_golden_vectors_match_oracle():
    d = np.load(os.path.join(GOLDEN, "quant_vectors.npz"))
    names = sorted({k.split("_", 1)[1] for k in d.files})
    for nm in names:
        q, s = fmt.quantize_rows(d["x_" + nm])
        assert np.array_equal(q, d["q_" + nm]) and np.array_equal(s, d["s_" + nm]), nm
        q2, s2 = cbuild.quantize_rows_c(d["x_" + nm])
        assert np.array_equal(q2, d["q_" + nm]) and np.array_equal(s2, d["s_" + nm]), nm


def test_bf16_round_matches_torch():
    import torch
    x = _rows(3, 16, 512)
    want = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(fmt.bf16_round(x), want)
