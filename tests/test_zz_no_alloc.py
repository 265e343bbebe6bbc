"""mxfp4_moe_decode_batch_noalloc (scratch in a fixed device array) against
mxfp4_moe_decode_batch (caller workspace), through the C ABI: the same
kernels, so the outputs must be identical bit for bit.  Two calls in a row,
the second with a smaller batch, so the second runs on a scratch that still
holds the first call's h; then the size limit is rejected on the host."""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import _lib
from moe_fused_inference_amd import moe_layer as ml
from tests.gpu_helpers import DEV, log

pytestmark = pytest.mark.gpu
H, MI, N_EXP = 2048, 768, 32


@pytest.fixture(scope="module")
def experts():
    g = torch.Generator(device=DEV)
    g.manual_seed(91)
    lib = _lib.load()

    def q(n, k):
        w = (torch.randn((N_EXP * n, k), generator=g, device=DEV) * 0.02).bfloat16()
        wp = torch.empty((N_EXP * n, k // 2), dtype=torch.uint8, device=DEV)
        ws = torch.empty((N_EXP * n, k // 32), dtype=torch.uint8, device=DEV)
        _lib.check(lib.mxfp4_prequant(w.data_ptr(), k, N_EXP * n, k, k, wp.data_ptr(), ws.data_ptr(), None), "q")
        return wp.view(N_EXP, n, k // 2), ws.view(N_EXP, n, k // 32)

    gwp, gws = q(MI, H)
    uwp, uws = q(MI, H)
    dwp, dws = q(H, MI)
    torch.cuda.synchronize()
    return ml.StackedExperts(gate_wp=gwp, gate_ws=gws, up_wp=uwp, up_ws=uws, down_wp=dwp, down_ws=dws)


def _inputs(M, E, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(N_EXP)[:E] for _ in range(M)]).astype(np.int32)
    w = rng.random((M, E)).astype(np.float32) + 0.05
    w /= w.sum(axis=1, keepdims=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = torch.randn((M, H), generator=g, device=DEV).bfloat16()
    lib = _lib.load()
    xq = torch.empty((M, H // 2), dtype=torch.uint8, device=DEV)
    xs = torch.empty((M, H // 32), dtype=torch.uint8, device=DEV)
    _lib.check(lib.mxfp4_prequant(x.data_ptr(), H, M, H, H, xq.data_ptr(), xs.data_ptr(), None), "prequant")
    return xq, xs, torch.from_numpy(ids).to(DEV), torch.from_numpy(w).to(DEV)


def _args(ex, xq, xs, ids, w, M, E, y):
    return (xq.data_ptr(), xs.data_ptr(), ids.data_ptr(), w.data_ptr(), ex.gate_wp.data_ptr(),
            ex.gate_ws.data_ptr(), ex.up_wp.data_ptr(), ex.up_ws.data_ptr(), ex.down_wp.data_ptr(),
            ex.down_ws.data_ptr(), N_EXP, M, E, H, MI, y.data_ptr())


def test_noalloc_equals_workspace_entry(experts):
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    for M, E, seed in ((16, 8, 1), (3, 4, 2)):    # the second call is smaller
        log(f"  noalloc vs workspace entry: M={M} E={E} seed={seed}")
        xq, xs, ids, w = _inputs(M, E, seed)
        y_ws = torch.full((M, H), float("nan"), device=DEV)
        y_na = torch.full((M, H), float("nan"), device=DEV)
        nb = lib.mxfp4_moe_decode_batch_workspace_size(M, E, MI)
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        _lib.check(lib.mxfp4_moe_decode_batch(*_args(experts, xq, xs, ids, w, M, E, y_ws), ws.data_ptr(), nb, st),
                   "moe_decode_batch")
        _lib.check(lib.mxfp4_moe_decode_batch_noalloc(*_args(experts, xq, xs, ids, w, M, E, y_na), st),
                   "moe_decode_batch_noalloc")
        torch.cuda.synchronize()
        assert torch.isfinite(y_ws).all()
        assert torch.equal(y_ws, y_na), f"M={M} E={E}: no-alloc output differs"


def test_noalloc_rejects_oversized_shapes(experts):
    lib = _lib.load()
    xq, xs, ids, w = _inputs(1, 8, 3)
    y = torch.empty((1, H), device=DEV)
    a = list(_args(experts, xq, xs, ids, w, 1, 8, y))
    a[14] = 4096   # Mi beyond the scratch's 2048
    assert lib.mxfp4_moe_decode_batch_noalloc(*a, None) == -1
    assert b"scratch" in lib.mxfp4_last_error()
    a[14] = MI
    a[11] = 17     # M beyond 16
    assert lib.mxfp4_moe_decode_batch_noalloc(*a, None) == -1
