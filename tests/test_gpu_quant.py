"""GPU parity of the activation quantizer: bit-exact against the oracle.

prequant   src/ext/mxfp4_decode.cu:24-50 (contract quant/fp4_format.py)
forward's activation quantization (fp16 rounding, src/ext/mxfp4_binding.cpp:31)
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import mxfp4 as fmt
from oracle import ops
from moe_fused_inference_amd import _lib
from tests.gpu_helpers import DEV, log, np_

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _check(dext, x_f32, what):
    xb = torch.from_numpy(x_f32).to(DEV).bfloat16()
    xq, xs = dext.prequant(xb)
    q, s = fmt.quantize_rows(np_(xb.float()))
    ok_q = np.array_equal(np_(xq), q)
    ok_s = np.array_equal(np_(xs), s)
    log(f"  prequant {what} {tuple(x_f32.shape)}: bytes_equal={ok_q} scales_equal={ok_s}")
    assert ok_s and ok_q, what


def test_prequant_golden_vectors(dext):
    d = np.load(os.path.join(GOLDEN, "quant_vectors.npz"))
    for nm in sorted({k.split("_", 1)[1] for k in d.files}):
        x = torch.from_numpy(d["x_" + nm]).to(DEV).bfloat16()
        xq, xs = dext.prequant(x)
        log(f"  golden {nm}")
        assert np.array_equal(np_(xq), d["q_" + nm]), nm
        assert np.array_equal(np_(xs), d["s_" + nm]), nm


@pytest.mark.parametrize("M,K", [(1, 64), (1, 2048), (3, 768), (2, 100), (2, 101), (9, 2048),
                                 (1, 1), (5, 33), (17, 4096), (4096, 2048)])
def test_prequant_shapes(dext, M, K):
    rng = np.random.default_rng(M * 7919 + K)
    x = rng.standard_normal((M, K)).astype(np.float32) * 0.5
    x[rng.random((M, K)) < 0.01] *= 4.0
    _check(dext, x, "random")


def test_prequant_every_bf16_pattern(dext):
    """Every finite bf16 value, (a) grouped 32 per block in a shuffled order
    and (b) alone in its block next to zeros (its own amax)."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    v = fmt.bf16_bits_to_f32(bits)
    v = v[np.isfinite(v)]
    rng = np.random.default_rng(11)
    pad = (-v.size) % 32
    grouped = np.concatenate([rng.permutation(v), np.zeros(pad, np.float32)]).reshape(-1, 32)
    _check(dext, grouped, "grouped")
    alone = np.zeros((v.size, 32), np.float32)
    alone[:, 5] = v
    _check(dext, alone, "alone")


def test_quantize_rows_every_f16_pattern(dext):
    """Every finite fp16 value through mxfp4_quantize_rows (fp16 input), grouped
    32 per block in a shuffled order and alone in its block: the quantizer's
    hardware E2M1 conversion on values with 11 significant bits."""
    lib = _lib.load()
    v = np.arange(1 << 16, dtype=np.uint16).view(np.float16)
    v = v[np.isfinite(v)].astype(np.float32)
    rng = np.random.default_rng(12)
    pad = (-v.size) % 32
    grouped = np.concatenate([rng.permutation(v), np.zeros(pad, np.float32)]).reshape(-1, 32)
    alone = np.zeros((v.size, 32), np.float32)
    alone[:, 9] = v
    for what, x in (("grouped", grouped), ("alone", alone)):
        xt = torch.from_numpy(x).to(DEV).half()
        M, K = xt.shape
        xq = torch.empty((M, K // 2), dtype=torch.uint8, device=DEV)
        xs = torch.empty((M, K // 32), dtype=torch.uint8, device=DEV)
        rc = lib.mxfp4_quantize_rows(xt.data_ptr(), 1, 0, K, M, K, K, xq.data_ptr(), xs.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        q, s = fmt.quantize_rows(np_(xt.float()))
        log(f"  quantize_rows every fp16 {what} {tuple(x.shape)}")
        assert np.array_equal(np_(xs), s), what
        assert np.array_equal(np_(xq), q), what


def test_prequant_edge_blocks(dext):
    rows = []
    r = np.zeros(96, np.float32)
    r[32:39] = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    r[39] = 6.0
    r[40:47] = [-0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5.0]
    r[64] = 96.0
    r[65:72] = -(2.0 ** -20)
    rows.append(r)
    r = np.zeros(96, np.float32)
    r[0] = 3 * 2.0 ** -126          # tiny amax (denormal-range quotient)
    r[1] = -(2.0 ** -133)
    r[32] = np.float32(3.0e38)      # scale code 253..254 territory
    r[33] = -np.float32(1.0e30)
    rows.append(r)
    _check(dext, np.stack(rows), "edges")


def test_prequant_strided_and_unaligned_input(dext):
    """Row stride > K and a 2-byte-aligned base take the element path."""
    lib = _lib.load()
    rng = np.random.default_rng(3)
    big = torch.from_numpy(rng.standard_normal((6, 200)).astype(np.float32)).to(DEV).bfloat16()
    for off, K in [(0, 150), (1, 150), (3, 64)]:
        view = big[:, off:off + K]
        M = view.shape[0]
        Kp = (K + 31) // 32 * 32
        xq = torch.empty((M, Kp // 2), dtype=torch.uint8, device=DEV)
        xs = torch.empty((M, Kp // 32), dtype=torch.uint8, device=DEV)
        rc = lib.mxfp4_prequant(view.data_ptr(), 200, M, K, Kp, xq.data_ptr(), xs.data_ptr(),
                                torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        q, s = fmt.quantize_rows(np_(view.float()))
        log(f"  strided off={off} K={K}")
        assert np.array_equal(np_(xq), q) and np.array_equal(np_(xs), s)


@pytest.mark.parametrize("src", ["bf16", "f16", "f32"])
def test_quantize_rows_dtypes_and_f16_rounding(dext, src):
    """mxfp4_quantize_rows on fp16/fp32 input, and the fp16 pre-rounding of
    `forward` (round_to_f16=1) on bf16/fp32 input."""
    lib = _lib.load()
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((7, 300)) * np.exp2(rng.integers(-20, 20, size=(7, 1)))).astype(np.float32)
    dt = {"bf16": (torch.bfloat16, 0), "f16": (torch.float16, 1), "f32": (torch.float32, 2)}[src]
    xt = torch.from_numpy(x).to(DEV).to(dt[0])
    xv = np_(xt.float())
    M, K = xt.shape
    Kp = 320
    for r16 in ([0, 1] if src != "f16" else [0]):
        xq = torch.empty((M, Kp // 2), dtype=torch.uint8, device=DEV)
        xs = torch.empty((M, Kp // 32), dtype=torch.uint8, device=DEV)
        rc = lib.mxfp4_quantize_rows(xt.data_ptr(), dt[1], r16, K, M, K, Kp, xq.data_ptr(), xs.data_ptr(),
                                     torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        q, s = (ops.forward_act_quant_ref(xv, Kp) if r16 else fmt.quantize_rows(xv, kp=Kp))
        log(f"  quantize_rows src={src} round_f16={r16}")
        assert np.array_equal(np_(xq), q) and np.array_equal(np_(xs), s)
