"""GPU parity of the batched decode MoE block (mxfp4_moe_decode_batch), the
two-launch replacement of forward_batch's moe_gateup -> moe_down ->
moe_combine chain (runtime/model_runner_v2.py:265-289).

Checked two ways on the same MXFP4 activations and stacked experts:
- against the drop-in chain on the GPU (route_tables + the _tab ops +
  moe_combine): g, u, the quantized h and every slot's down product are the
  same arithmetic in the same order, so only the combine's fp32 summation
  order differs (cos >= 0.9999999, max-rel <= 1e-5);
- against the oracle (oracle/ops.py: moe_gateup_ref, moe_down_ref with the
  GPU's own h, moe_combine_ref) at the per-op bar.
Routing covers shared experts (several tokens on one expert), a token set
whose slots all hit distinct experts, M = 1 and the 16-token maximum, and ids
outside [0, n_experts), which contribute nothing.
"""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import _lib
from moe_fused_inference_amd import moe_layer as ml
from oracle import mxfp4 as fmt
from oracle import ops
from tests.gpu_helpers import DEV, assert_close, log, np_

pytestmark = pytest.mark.gpu
H, MI, N_EXP, E = 2048, 768, 32, 8


@pytest.fixture(scope="module")
def experts():
    g = torch.Generator(device=DEV)
    g.manual_seed(77)
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


def _routing(M, mode, seed):
    rng = np.random.default_rng(seed)
    if mode == "shared":        # few popular experts: most experts serve several tokens
        pool = rng.permutation(N_EXP)[:12]
        ids = np.stack([rng.choice(pool, E, replace=False) for _ in range(M)])
    elif mode == "distinct":    # every slot a different expert (M * E <= N_EXP)
        ids = rng.permutation(N_EXP)[:M * E].reshape(M, E)
    else:                       # uniform, with a few ids outside [0, n_experts)
        ids = np.stack([rng.permutation(N_EXP)[:E] for _ in range(M)])
        ids[0, 3] = -1
        ids[M - 1, 5] = N_EXP + 2
    w = rng.random((M, E)).astype(np.float32) + 0.05
    w /= w.sum(axis=1, keepdims=True)
    return ids.astype(np.int32), w


def _dropin(ex, xq, xs, ids, w, M):
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    idc = torch.from_numpy(np.clip(ids, 0, N_EXP - 1)).to(DEV)   # route_tables clamps; masked below
    tabs = [torch.empty(M * 2 * E if i < 2 else M * E, dtype=torch.int64, device=DEV) for i in range(4)]
    _lib.check(lib.mxfp4_route_tables(idc.data_ptr(), M, E, ex.gate_wp.data_ptr(), ex.gate_ws.data_ptr(),
                                      ex.up_wp.data_ptr(), ex.up_ws.data_ptr(), ex.down_wp.data_ptr(),
                                      ex.down_ws.data_ptr(), N_EXP, H, MI, *[t.data_ptr() for t in tabs], st), "tab")
    gu = torch.empty((M * E, 2 * MI), dtype=torch.float32, device=DEV)
    yd = torch.empty((M * E, H), dtype=torch.float32, device=DEV)
    _lib.check(lib.mxfp4_moe_gateup_devtab(xq.data_ptr(), xs.data_ptr(), tabs[0].data_ptr(), tabs[1].data_ptr(),
                                           gu.data_ptr(), E, M, MI, H, H, st), "gateup")
    _lib.check(lib.mxfp4_moe_down_devtab(gu.data_ptr(), tabs[2].data_ptr(), tabs[3].data_ptr(), yd.data_ptr(), E, M,
                                         H, MI, MI, st), "down")
    valid = torch.from_numpy(((ids >= 0) & (ids < N_EXP)).astype(np.float32)).to(DEV)
    wt = torch.from_numpy(w).to(DEV) * valid                      # invalid ids contribute nothing
    out = torch.empty((M, H), dtype=torch.float32, device=DEV)
    _lib.check(lib.mxfp4_moe_combine(yd.data_ptr(), H, wt.contiguous().data_ptr(), E, out.data_ptr(), M, H, st),
               "combine")
    return out, gu, yd


@pytest.mark.parametrize("M,mode", [(1, "uniform"), (4, "shared"), (8, "shared"), (8, "uniform"), (9, "shared"),
                                    (4, "distinct"), (16, "shared")])
def test_decode_batch_matches_dropin_and_oracle(experts, M, mode):
    ex = experts
    g = torch.Generator(device=DEV)
    g.manual_seed(M * 10 + len(mode))
    x = torch.randn((M, H), generator=g, device=DEV).bfloat16()
    xq = torch.empty((M, H // 2), dtype=torch.uint8, device=DEV)
    xs = torch.empty((M, H // 32), dtype=torch.uint8, device=DEV)
    lib = _lib.load()
    _lib.check(lib.mxfp4_prequant(x.data_ptr(), H, M, H, H, xq.data_ptr(), xs.data_ptr(), None), "prequant")
    ids, w = _routing(M, mode, seed=M + 100)
    idt, wt = torch.from_numpy(ids).to(DEV), torch.from_numpy(w).to(DEV)
    y = ml.decode_batch(xq, xs, idt, wt, ex)
    ref, gu, yd = _dropin(ex, xq, xs, ids, w, M)
    torch.cuda.synchronize()
    what = f"M={M} {mode}"
    assert_close(np_(y), np_(ref), 0.9999999, 1e-5, what=f"{what} vs drop-in chain")
    # oracle on the GPU's h (the quantizer's input), as the moe_down tests do
    xqn, xsn = np_(xq), np_(xs)
    valid = (ids >= 0) & (ids < N_EXP)
    ic = np.clip(ids, 0, N_EXP - 1)
    gw = [np_(ex.gate_wp[int(e)]) if p == 0 else np_(ex.up_wp[int(e)]) for m in range(M) for p in (0, 1)
          for e in ic[m]]
    gs = [np_(ex.gate_ws[int(e)]) if p == 0 else np_(ex.up_ws[int(e)]) for m in range(M) for p in (0, 1)
          for e in ic[m]]
    gu_ref = ops.moe_gateup_ref(xqn, xsn, gw, gs, E, M, MI)
    assert_close(np_(gu), gu_ref, what=f"{what} gate/up")
    h = ops.moe_down_h_ref(np_(gu), E, M, MI)
    yd_ref = ops.moe_down_ref(np_(gu), [np_(ex.down_wp[int(e)]) for e in ic.reshape(-1)],
                              [np_(ex.down_ws[int(e)]) for e in ic.reshape(-1)], E, M, H, MI, h=h)
    out_ref = ops.moe_combine_ref(yd_ref, (w * valid).astype(np.float32), M)
    assert_close(np_(y), out_ref, what=f"{what} vs oracle")
    log(f"  {what}: distinct experts {len(set(ic[valid].tolist()))}")


def test_decode_batch_graph_replays(experts):
    """Captured once, replayed with new activations: equal to eager calls."""
    ex = experts
    M = 8
    ids, w = _routing(M, "shared", seed=5)
    idt, wt = torch.from_numpy(ids).to(DEV), torch.from_numpy(w).to(DEV)
    xq = torch.zeros((M, H // 2), dtype=torch.uint8, device=DEV)
    xs = torch.full((M, H // 32), 127, dtype=torch.uint8, device=DEV)
    out = torch.empty((M, H), dtype=torch.float32, device=DEV)
    lib = _lib.load()
    ws = torch.empty(lib.mxfp4_moe_decode_batch_workspace_size(M, E, MI), dtype=torch.uint8, device=DEV)
    ml.decode_batch(xq, xs, idt, wt, ex, out=out, ws=ws)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            ml.decode_batch(xq, xs, idt, wt, ex, out=out, ws=ws)
    torch.cuda.synchronize()
    g = torch.Generator(device=DEV)
    for rep in range(3):
        g.manual_seed(rep)
        xq.copy_(torch.randint(0, 256, xq.shape, generator=g, device=DEV, dtype=torch.uint8))
        xs.copy_(torch.randint(118, 128, xs.shape, generator=g, device=DEV, dtype=torch.uint8))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = ml.decode_batch(xq, xs, idt, wt, ex)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"


def test_decode_batch_argument_checks(experts):
    lib = _lib.load()
    ex = experts
    buf = torch.empty(1 << 16, dtype=torch.uint8, device=DEV)
    p = buf.data_ptr()
    args = [p, p, p, p, ex.gate_wp.data_ptr(), ex.gate_ws.data_ptr(), ex.up_wp.data_ptr(), ex.up_ws.data_ptr(),
            ex.down_wp.data_ptr(), ex.down_ws.data_ptr(), N_EXP]
    assert lib.mxfp4_moe_decode_batch(*args, 17, E, H, MI, p, p, 1 << 16, None) == -1
    assert "M=17" in lib.mxfp4_last_error().decode()
    assert lib.mxfp4_moe_decode_batch(*args, 2, 9, H, MI, p, p, 1 << 16, None) == -1
    assert "E=9" in lib.mxfp4_last_error().decode()
    assert lib.mxfp4_moe_decode_batch(*args, 2, E, 2000, MI, p, p, 1 << 16, None) == -1
    assert "H=2000" in lib.mxfp4_last_error().decode()
    assert lib.mxfp4_moe_decode_batch(*args, 2, E, H, MI, p, p, 16, None) == -1
    assert "workspace" in lib.mxfp4_last_error().decode()
