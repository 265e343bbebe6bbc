"""Pins oracle/step.py's RMSNorm and RoPE restatements.

Against torch-CPU evaluations of the reference's formulas
(runtime/model_runner.py:20-41 is written in torch ops; torch's CPU kernels
are an independent implementation of the same arithmetic) and against
closed forms: RoPE at position 0 is the identity, a rotation keeps the norm
of every (i, i + D/2) pair, and RMSNorm of a constant row is the weight.
"""
import numpy as np
import torch

from oracle import mxfp4 as fmt
from oracle import step as sref


def torch_rms_norm(x, w, eps):
    dtype = x.dtype
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return (xf.to(dtype)) * w


def torch_rope(x, positions, theta):
    D = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    freqs = positions.float()[:, None] * inv[None, :]
    cos = torch.cat([freqs.cos(), freqs.cos()], dim=-1)[:, None]
    sin = torch.cat([freqs.sin(), freqs.sin()], dim=-1)[:, None]
    x1, x2 = x.chunk(2, dim=-1)
    rot = torch.cat((-x2, x1), dim=-1)
    return (x * cos + rot * sin).to(x.dtype)


def test_rms_norm_matches_torch_bf16():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn((16, 2048), generator=g) * 3).bfloat16()
    w = (1 + 0.1 * torch.randn(2048, generator=g)).bfloat16()
    want = torch_rms_norm(x, w, 1e-6).float().numpy()
    got = sref.rms_norm_ref(x.float().numpy(), w.float().numpy(), 1e-6)
    # the fp32 mean differs from torch's in the last bit at most: a bf16
    # result may round the other way, never by more than one bf16 ulp
    assert np.mean(got == want) > 0.995
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= 2 ** -7


def test_rms_norm_fp32_head_norm_matches_torch():
    g = torch.Generator().manual_seed(1)
    q = torch.randn((3, 4, 128), generator=g) * 5
    w = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    want = torch_rms_norm(q, w, 1e-6).bfloat16().float().numpy()
    got = sref.rms_norm_ref(q.numpy(), w.float().numpy(), 1e-6, bf16_input=False)
    assert np.mean(got == want) > 0.995
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= 2 ** -7


def test_rms_norm_constant_row_is_the_weight():
    w = fmt.bf16_round(np.linspace(0.5, 1.5, 2048).astype(np.float32))
    for c in (3.0, -0.25, 1000.0):
        got = sref.rms_norm_ref(np.full((1, 2048), c, np.float32), w, 1e-6)
        assert np.array_equal(got[0], np.sign(c) * w)


def test_rope_matches_torch_and_closed_forms():
    g = torch.Generator().manual_seed(2)
    x = torch.randn((5, 4, 128), generator=g).bfloat16()
    pos = torch.tensor([0, 1, 7, 1000, 4095])
    want = torch_rope(x, pos, 1e6).float().numpy()
    got = sref.rope_ref(x.float().numpy(), pos.numpy(), 1e6)
    assert np.mean(got == want) > 0.99
    assert np.max(np.abs(got - want)) <= 2 ** -6 * np.max(np.abs(want))
    # position 0: identity
    assert np.array_equal(got[0], x[0].float().numpy())
    # each (i, i + 64) pair is rotated: its norm is kept up to bf16 rounding
    xf = x.float().numpy()
    n_in = np.hypot(xf[..., :64], xf[..., 64:])
    n_out = np.hypot(got[..., :64], got[..., 64:])
    assert np.max(np.abs(n_out - n_in) / np.maximum(n_in, 1e-3)) < 2 ** -6


def test_embed_ref_is_dequant():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((10, 64)).astype(np.float32)
    wp, ws = fmt.quantize_rows(w)
    got = sref.embed_ref(wp, ws, [3, 0, 3], 64)
    deq = fmt.dequant_rows(wp, ws, 64)
    assert np.array_equal(got, deq[[3, 0, 3]])   # E2M1 x 2^k is exact in bf16


def test_argmax_ref_first_maximum():
    lg = np.array([[1.0, 5.0, 5.0], [-1.0, -1.0, -2.0]])
    assert sref.argmax_ref(lg).tolist() == [1, 0]
