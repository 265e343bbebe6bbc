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


def _capture_child(root):
    """Body of the fresh process: the process's first two no-alloc calls are
    made inside a HIP graph capture (so the per-device scratch lookup runs
    during capture), the graph is replayed with eager work in between, and
    every replay is compared with the workspace entry point."""
    import sys
    sys.path.insert(0, root)
    lib = _lib.load()
    g = torch.Generator(device=DEV)
    g.manual_seed(92)

    def q(n, k):
        w = (torch.randn((8 * n, k), generator=g, device=DEV) * 0.02).bfloat16()
        wp = torch.empty((8 * n, k // 2), dtype=torch.uint8, device=DEV)
        ws = torch.empty((8 * n, k // 32), dtype=torch.uint8, device=DEV)
        _lib.check(lib.mxfp4_prequant(w.data_ptr(), k, 8 * n, k, k, wp.data_ptr(), ws.data_ptr(), None), "q")
        return wp.view(8, n, k // 2), ws.view(8, n, k // 32)

    gwp, gws = q(MI, H)
    uwp, uws = q(MI, H)
    dwp, dws = q(H, MI)
    ex = ml.StackedExperts(gate_wp=gwp, gate_ws=gws, up_wp=uwp, up_ws=uws, down_wp=dwp, down_ws=dws)
    calls = []
    for M, E, seed in ((4, 8, 5), (2, 4, 6)):
        rng = np.random.default_rng(seed)
        ids = torch.from_numpy(np.stack([rng.permutation(8)[:E] for _ in range(M)]).astype(np.int32)).to(DEV)
        w = rng.random((M, E)).astype(np.float32) + 0.05
        w = torch.from_numpy(w / w.sum(axis=1, keepdims=True)).to(DEV)
        x = torch.randn((M, H), generator=g, device=DEV).bfloat16()
        xq = torch.empty((M, H // 2), dtype=torch.uint8, device=DEV)
        xs = torch.empty((M, H // 32), dtype=torch.uint8, device=DEV)
        _lib.check(lib.mxfp4_prequant(x.data_ptr(), H, M, H, H, xq.data_ptr(), xs.data_ptr(), None), "prequant")
        a = (xq.data_ptr(), xs.data_ptr(), ids.data_ptr(), w.data_ptr(), ex.gate_wp.data_ptr(), ex.gate_ws.data_ptr(),
             ex.up_wp.data_ptr(), ex.up_ws.data_ptr(), ex.down_wp.data_ptr(), ex.down_ws.data_ptr(), 8, M, E, H, MI)
        calls.append((M, E, a, (xq, xs, ids, w), torch.full((M, H), float("nan"), device=DEV)))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            st = torch.cuda.current_stream().cuda_stream
            for M, E, a, _, y in calls:
                _lib.check(lib.mxfp4_moe_decode_batch_noalloc(*a, y.data_ptr(), st), "noalloc under capture")
    torch.cuda.synchronize()
    st = torch.cuda.current_stream().cuda_stream
    refs = []
    for M, E, a, _, _ in calls:
        y = torch.full((M, H), float("nan"), device=DEV)
        nb = lib.mxfp4_moe_decode_batch_workspace_size(M, E, MI)
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        _lib.check(lib.mxfp4_moe_decode_batch(*a, y.data_ptr(), ws.data_ptr(), nb, st), "moe_decode_batch")
        refs.append(y)
    torch.cuda.synchronize()
    for rep in range(3):
        for _, _, _, _, y in calls:
            y.fill_(float("nan"))
        _ = torch.randn(4096, device=DEV).sum().item()   # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for (M, E, _, _, y), ref in zip(calls, refs):
            assert torch.isfinite(ref).all()
            assert torch.equal(y, ref), f"replay {rep}: M={M} E={E} no-alloc under capture differs"
    print("capture ok", flush=True)


def test_noalloc_first_call_under_graph_capture():
    """In a fresh process (so the no-alloc entry's per-device scratch lookup
    has not run yet), the first two calls are recorded in a HIP graph; every
    replay equals the workspace entry point bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path.insert(0, %r); from tests import test_zz_no_alloc as t; t._capture_child(%r)"
            % (root, root))
    log("  fresh process: first no-alloc calls inside a graph capture")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240, cwd=root)
    log(r.stdout[-2000:])
    assert r.returncode == 0, r.stderr[-4000:]
    assert "capture ok" in r.stdout
