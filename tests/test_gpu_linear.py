"""GPU parity of the block-scaled linear operators against the oracle.

lin_pq   src/ext/mxfp4_decode.cu:135-170   (grouped GEMV for M <= 16, MFMA GEMM above)
forward  src/ext/mxfp4_linear.cu:106-198   (fp16 rounding + quantize + GEMM)

Tolerances: per-op (same quantized operands) cos >= 0.99999, max-rel <= 1e-4
(tests/gpu_helpers.py), tighter than the north-star cos >= 0.999 / 1e-2.
"""
import numpy as np
import pytest
import torch

from oracle import mxfp4 as fmt
from oracle import ops
from moe_fused_inference_amd import _lib
from tests.gpu_helpers import DEV, assert_close, log, np_

pytestmark = pytest.mark.gpu


def _w(dext, N, K, seed):
    rng = np.random.default_rng(seed)
    W = rng.standard_normal((N, K)).astype(np.float32)
    W *= np.power(2.0, rng.integers(-1, 2, size=(N, 1))).astype(np.float32)
    wq, ws = fmt.quantize_rows(W)
    return torch.from_numpy(wq).to(DEV), torch.from_numpy(ws).to(DEV), wq, ws


# shapes of tests/correctness/test_mxfp4_decode.py:78-79 plus GEMM-path shapes
LIN_SHAPES = [(1, 32, 64), (1, 768, 2048), (1, 2048, 768), (3, 128, 100), (1, 4096, 2048),
              (2, 2048, 2048), (16, 64, 96), (17, 64, 256), (128, 128, 256), (200, 300, 1000),
              (129, 257, 40), (512, 1536, 2048), (300, 520, 768), (2048, 2048, 768),
              (2048, 4096, 512), (2000, 4000, 768),   # these two on the 256 x 256 tile GEMM
              # ragged edges on the 128 x 128 ring (192 tiles) and the 4-stage 64 x 64 ring (270 tiles);
              # (512, 1536, 2048), (17, 64, 256) and (300, 520, 768) run on the 8-stage 64 x 64 ring
              (1000, 3000, 512), (1100, 900, 1024),
              # small-M split-K GEMV: K in 16 / 8 / 4 parts, unsplit with 4 row tiles, odd step count
              (1, 128, 2048), (1, 2048, 4096), (1, 5120, 2048), (3, 20000, 2048), (5, 1000, 4160),
              (8, 136, 2048), (40, 48, 96)]


@pytest.mark.parametrize("M,N,K", LIN_SHAPES)
def test_lin_pq_vs_oracle(dext, M, N, K):
    rng = np.random.default_rng(M + N + K)
    wp, wsc, wq, ws = _w(dext, N, K, seed=N * 31 + K)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32) * 0.5).to(DEV).bfloat16()
    xq, xs = dext.prequant(x)
    y = dext.lin_pq(xq, xs, wp, wsc, M, N, K)
    torch.cuda.synchronize()
    ref = ops.lin_pq_ref(np_(xq), np_(xs), wq, ws)
    assert y.shape == (M, N) and y.dtype == torch.float32
    assert_close(np_(y), ref, what=f"lin_pq M={M} N={N} K={K}")


# shapes of tests/correctness/test_mxfp4_mma.py:74-100 plus config-3 shapes
FWD_SHAPES = [(16, 8, 64), (16, 8, 100), (16, 8, 40), (1, 8, 64), (1, 32, 64), (16, 32, 64),
              (32, 32, 64), (8, 64, 2048), (1, 768, 2048), (8, 2048, 768), (2048, 2048, 768)]


@pytest.mark.parametrize("M,N,K", FWD_SHAPES)
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_forward_vs_oracle(lext, M, N, K, xdt):
    rng = np.random.default_rng(M * 3 + N * 5 + K)
    wp, wsc, wq, ws = _w(None, N, K, seed=N + K)
    x = rng.standard_normal((M, K)).astype(np.float32) * 0.5
    x[rng.random((M, K)) < 0.005] *= 4.0
    xt = torch.from_numpy(x).to(DEV).to(xdt)
    y = lext.forward(xt, wp, wsc)
    torch.cuda.synchronize()
    ref = ops.forward_ref(np_(xt.float()), wq, ws)
    assert_close(np_(y), ref, what=f"forward {xdt} M={M} N={N} K={K}")


def test_forward_equals_prequant_then_lin_pq(dext, lext):
    """Structural: forward == quantize(fp16(x)) then lin_pq, bit for bit."""
    rng = np.random.default_rng(9)
    M, N, K = 64, 512, 2048
    wp, wsc, _, _ = _w(dext, N, K, seed=5)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(DEV).half()
    y1 = lext.forward(x, wp, wsc)
    lib = _lib.load()
    Kp = 2048
    xq = torch.empty((M, Kp // 2), dtype=torch.uint8, device=DEV)
    xs = torch.empty((M, Kp // 32), dtype=torch.uint8, device=DEV)
    assert lib.mxfp4_quantize_rows(x.data_ptr(), 1, 1, K, M, K, Kp, xq.data_ptr(), xs.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream) == 0
    y2 = dext.lin_pq(xq, xs, wp, wsc, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


def test_config3_largest_gemm_north_star(lext):
    """(4096, 4096, 2048), activations bf16 N(0,1) quantized on the fly, weights
    MXFP4 from bf16 N(0,0.02): per-op tolerance against the oracle."""
    M, N, K = 4096, 4096, 2048
    g = torch.Generator(device=DEV)
    g.manual_seed(30)
    x = torch.randn((M, K), generator=g, device=DEV).bfloat16()
    w = (torch.randn((N, K), generator=g, device=DEV) * 0.02).bfloat16()
    wq, ws = fmt.quantize_rows(np_(w.float()))
    y = lext.forward(x, torch.from_numpy(wq).to(DEV), torch.from_numpy(ws).to(DEV))
    torch.cuda.synchronize()
    ref = ops.forward_ref(np_(x.float()), wq, ws)
    assert_close(np_(y), ref, what="forward 4096x4096x2048")
