"""Bit-identity of the RMSNorm wave sum (mx::wave_sum_butterfly: permlane32 /
permlane16 swaps, a row rotation and quad / half-row DPP moves) with the plain
__shfl_xor butterfly (xor 32, 16, 8, 4, 2, 1), on every lane of every wave:
random, mixed-magnitude (cancellation-heavy), subnormal and inf / NaN waves.
The fused and separate norm kernels all use the butterfly, so this is the test
that ties it to the shuffle order the reduction is specified by."""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import _lib
from tests.gpu_helpers import DEV, log

pytestmark = pytest.mark.gpu


def _waves(rng):
    w = []
    w.append(rng.standard_normal((256, 64)))
    # mixed magnitudes: each lane scaled by 2^e, e in [-60, 60]
    w.append(rng.standard_normal((256, 64)) * np.exp2(rng.integers(-60, 61, (256, 64))))
    # near-cancelling pairs
    a = rng.standard_normal((128, 32)) * 1e4
    w.append(np.concatenate([a, -a + rng.standard_normal((128, 32)) * 1e-3], axis=1))
    # subnormals and zeros of both signs
    sub = rng.integers(-(2 ** 22), 2 ** 22, (64, 64)).astype(np.int64)
    w.append(np.where(sub < 0, -1.0, 1.0) * (np.abs(sub).astype(np.float64) * 2.0 ** -149))
    w.append(np.where(rng.random((16, 64)) < 0.5, 0.0, -0.0))
    # inf / -inf / NaN (the default quiet NaN only, so any propagation order gives its bits)
    s = rng.standard_normal((64, 64))
    for k in range(64):
        j = rng.integers(0, 64, 3)
        s[k, j[0]] = np.inf if k % 3 else -np.inf
        if k % 4 == 1:
            s[k, j[1]] = -np.inf
        if k % 5 == 2:
            s[k, j[2]] = np.nan
    w.append(s)
    return np.concatenate(w).astype(np.float32)


def test_wave_sum_butterfly_bits_equal_shfl_xor():
    lib = _lib.load()
    x = torch.from_numpy(_waves(np.random.default_rng(77))).to(DEV).contiguous()
    n = x.shape[0]
    a = torch.empty_like(x)
    b = torch.empty_like(x)
    _lib.check(lib.mxfp4_selftest_wave_sum(x.data_ptr(), a.data_ptr(), b.data_ptr(), n,
                                           torch.cuda.current_stream().cuda_stream), "selftest_wave_sum")
    torch.cuda.synchronize()
    ai, bi = a.view(torch.int32), b.view(torch.int32)
    bad = (ai != bi).sum().item()
    log(f"  {n} waves, {int(torch.isnan(b).any(1).sum())} with NaN sums, {int(torch.isinf(b).any(1).sum())} with inf: "
        f"{bad} lanes differ")
    assert bad == 0
    # every lane of a wave holds the same sum, and it is the fp32 sum of the wave in some order
    assert bool((bi == bi[:, :1]).all())
    fin = torch.isfinite(b[:, 0])
    ref = x.double().sum(1)
    err = (b[fin, 0].double() - ref[fin]).abs() / x[fin].double().abs().sum(1).clamp_min(1e-300)
    assert float(err.max()) < 1e-5
