"""Pins of the attention / KV-cache oracle (oracle/attn.py) on the CPU.

The reference's KV byte codec (src/ext/mxfp4_decode.cu:355-364,437-455) is
checked against torch's OCP float8_e4m3fn where the two definitions agree
(normal codes, away from rounding ties) and against closed forms where they
differ on purpose (ties rounded away from zero, the subnormal and
saturation rules); the attention oracle against special cases whose answer
is known without it.
"""
import numpy as np
import pytest
import torch

from oracle import attn


def _all_finite_bf16():
    b = np.arange(65536, dtype=np.uint32)
    f = (b << 16).view(np.float32)
    return f[np.isfinite(f)]


def test_decode_matches_ocp_on_normal_codes_and_closed_forms_elsewhere():
    codes = np.arange(256, dtype=np.uint8)
    got = attn.e4m3_ref_decode(codes)
    ocp = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    e = (codes >> 3) & 15
    m = (codes & 7).astype(np.float64)
    sgn = np.where(codes & 0x80, -1.0, 1.0)
    normal = (e >= 1) & (e <= 14)
    assert np.array_equal(got[normal], ocp[normal])
    assert np.array_equal(got[e == 0], (sgn * m * 2.0 ** -6)[e == 0].astype(np.float32))
    assert np.array_equal(got[e == 15], (sgn * 448.0 * (1 + m / 8))[e == 15].astype(np.float32))


def test_encode_against_ocp_rne_and_closed_forms():
    v = _all_finite_bf16()
    got = attn.e4m3_ref_encode(v)
    a = np.abs(v).astype(np.float64)
    sign = np.where(v < 0, 0x80, 0)
    ocp = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # normal range below the saturation point: OCP round-to-nearest-even except at ties
    rng = (a >= 2.0 ** -6) & (a < 248.0)
    differ = rng & (got != ocp)
    man = a / np.exp2(np.floor(np.log2(np.where(a > 0, a, 1.0))))
    frac = (man - 1.0) * 8.0
    tie = np.abs(frac - np.floor(frac) - 0.5) == 0
    assert differ.any() and (tie[differ]).all(), "codes differ only at exact ties"
    dec = np.abs(attn.e4m3_ref_decode(got).astype(np.float64))
    assert (dec[differ] > a[differ]).all(), "ties go away from zero"
    assert (np.abs(attn.e4m3_ref_decode(got[rng]) - v[rng]) <= np.abs(
        torch.from_numpy(ocp[rng]).view(torch.float8_e4m3fn).float().numpy() - v[rng]) + 1e-30).all()
    # below 2^-6: a mantissa that rounds up to 2 carries into the normal code
    # 0x08 (= 2^-6) before the subnormal rule; otherwise lroundf(a * 64): 0 / 1
    small = (a > 0) & (a < 2.0 ** -6)
    want = np.where(a >= 2.0 ** -7 * 1.9375, 8, (a >= 2.0 ** -7).astype(np.int64))
    assert np.array_equal(got[small], (sign | want)[small].astype(np.uint8))
    # zero keeps its sign; at and above 248 everything saturates to 0x7F
    assert np.array_equal(got[a == 0], sign[a == 0].astype(np.uint8))
    big = a >= 248.0
    assert np.array_equal(got[big], (sign | 0x7F)[big].astype(np.uint8))


def test_encode_round_trips_normal_codes():
    codes = np.array([c for c in range(256) if 1 <= (c >> 3) & 15 <= 14], np.uint8)
    assert np.array_equal(attn.e4m3_ref_encode(attn.e4m3_ref_decode(codes)), codes)


def _cache(rng, max_pos, Hkv, D, scale=1.0):
    return attn.e4m3_ref_encode(rng.standard_normal((max_pos, Hkv, D)).astype(np.float32) * scale)


def test_attn_single_position_returns_v0():
    rng = np.random.default_rng(1)
    kvk, kvv = _cache(rng, 8, 2, 128), _cache(rng, 8, 2, 128)
    q = rng.standard_normal((1, 4, 128)).astype(np.float32)
    o, sc = attn.attn_decode_ref(q, kvk, kvv, base=0)
    vd = attn.e4m3_ref_decode(kvv).astype(np.float64)
    for h in range(4):
        assert np.array_equal(o[0, h], vd[0, h // 2])
    assert sc[0].shape == (4, 1)


def test_attn_zero_query_is_mean_of_values_and_scores_are_dots():
    rng = np.random.default_rng(2)
    kvk, kvv = _cache(rng, 64, 4, 128), _cache(rng, 64, 4, 128)
    q = np.zeros((2, 8, 128), np.float32)
    q[1] = rng.standard_normal((8, 128))
    o, sc = attn.attn_decode_ref(q, kvk, kvv, base=20)
    vd = attn.e4m3_ref_decode(kvv).astype(np.float64)
    kd = attn.e4m3_ref_decode(kvk).astype(np.float64)
    for h in range(8):
        assert np.allclose(o[0, h], vd[:21, h // 2].mean(0), rtol=1e-12, atol=1e-12)
        assert np.allclose(sc[1][h], np.array([kd[s, h // 2] @ q[1, h] for s in range(22)]), rtol=1e-12)


def test_attn_dominant_key_selects_its_value_and_out_of_range_rows():
    rng = np.random.default_rng(3)
    kvk, kvv = _cache(rng, 16, 1, 128), _cache(rng, 16, 1, 128)
    kd = attn.e4m3_ref_decode(kvk).astype(np.float64)
    q = (kd[5, 0] * 50.0).astype(np.float32)[None, None, :]
    o, _ = attn.attn_decode_ref(q, kvk, kvv, base=15)
    assert np.allclose(o[0, 0], attn.e4m3_ref_decode(kvv)[5, 0], atol=1e-6)
    o, sc = attn.attn_decode_ref(np.zeros((3, 1, 128), np.float32), kvk, kvv, base=14)
    assert sc[2] is None and np.isnan(o[2]).all() and not np.isnan(o[1]).any()


def test_kv_write_ref_rows():
    rng = np.random.default_rng(4)
    k = rng.standard_normal((3, 2, 128)).astype(np.float32)
    v = rng.standard_normal((3, 2, 128)).astype(np.float32)
    kvk = np.zeros((10, 2, 128), np.uint8)
    kvv = np.zeros((10, 2, 128), np.uint8)
    attn.kv_write_ref(k, v, kvk, kvv, base=8)
    assert np.array_equal(kvk[8], attn.e4m3_ref_encode(k[0])) and np.array_equal(kvv[9], attn.e4m3_ref_encode(v[1]))
    assert not kvk[:8].any()


def test_torch_encode_matches_torch_on_every_bf16_pattern():
    """e4m3_torch_encode is torch's float -> float8_e4m3fn conversion, the
    reference batch step's cache write: identical bytes on all 65536 bf16 bit
    patterns (NaNs, infinities, subnormals, both zeros) and on random fp32."""
    allv = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float().numpy()
    want = torch.from_numpy(allv).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = attn.e4m3_torch_encode(allv)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]
    rng = np.random.default_rng(0)
    f = (rng.standard_normal(200000) * np.exp2(rng.integers(-12, 10, 200000))).astype(np.float32)
    f[:6] = [464.0, 464.00003, -464.0, 479.9, 2.0 ** -7 * 1.5, 2.0 ** -10]   # tie to 448, past it, subnormal ties
    want = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(attn.e4m3_torch_encode(f), want)
    # and the closed forms: 448 is the largest finite code, ties go to the even mantissa
    assert attn.e4m3_torch_encode(np.float32([448.0, 456.0, 1.0625, 1.1875]))[0:4].tolist() == [0x7E, 0x7E, 0x38, 0x3A]
