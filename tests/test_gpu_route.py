"""GPU parity of the device routing (mxfp4_route_topk, mxfp4_route_tables):
the host-side softmax -> top-k -> renormalise and the token-major pointer
tables of runtime/model_runner_v2.py:189-202 / :272-286, as kernels.

Oracle: oracle.ops.route_topk_np (numpy restatement, pinned against the
reference's own torch calls in tests/test_oracle_ops.py) and
oracle.ops.route_ref (those torch calls on CPU).  Ids must match exactly
(the random logits have no exact probability ties); weights within 2e-6 of
the largest weight (the device exp and the host exp may differ by an ulp).
The tables must drive the drop-in grouped ops to the same bits as the host
pointer lists, and the fused layer with device routing must equal host
routing, also inside a replayed HIP graph.
"""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import moe_layer
from oracle import ops
from tests.gpu_helpers import DEV, log, np_, rand_weight

pytestmark = pytest.mark.gpu
W_TOL = 2e-6


def _logits(M, n, seed, scale=3.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((M, n)) * scale).astype(np.float32)


@pytest.mark.parametrize("M,n,k,norm", [(1, 128, 8, True), (9, 128, 8, True), (300, 128, 8, True),
                                        (64, 60, 1, True), (33, 256, 32, False), (17, 1024, 8, True),
                                        (5, 8, 8, True), (3, 200, 5, False)])
def test_route_topk_vs_oracle(M, n, k, norm):
    lg = _logits(M, n, seed=M * 1000 + n + k)
    ids, w, ids64 = moe_layer.route_topk(torch.from_numpy(lg).to(DEV), k, norm=norm, want_int64=True)
    torch.cuda.synchronize()
    ti, tv = ops.route_topk_np(lg, k, renorm=norm)
    assert np.array_equal(np_(ids), ti), "ids differ from the oracle"
    assert np.array_equal(np_(ids64), ti)
    err = float(np.abs(np_(w) - tv).max() / np.abs(tv).max())
    log(f"  route_topk M={M} n={n} k={k} norm={norm}: ids exact, weight err {err:.2e}")
    assert err <= W_TOL
    ri, _ = ops.route_ref(lg, k, renorm=norm)          # the reference's torch calls
    assert np.array_equal(np_(ids), ri)


def test_route_topk_special_rows():
    n, k = 64, 4
    lg = np.zeros((4, n), np.float32)                  # row 0: all equal -> 0..3, weights 1/4
    lg[1, :] = -np.inf                                  # row 1: masked experts
    lg[1, [40, 3, 17, 55, 9]] = [1.0, 5.0, 2.0, 3.0, -1.0]
    lg[2, 50] = 60.0                                    # row 2: one dominant logit
    lg[3] = np.arange(n, dtype=np.float32)[::-1] * 1e-3  # row 3: strictly descending by index
    ids, w = moe_layer.route_topk(torch.from_numpy(lg).to(DEV), k)
    torch.cuda.synchronize()
    ti, tv = ops.route_topk_np(lg, k)
    assert np.array_equal(np_(ids), ti)
    assert np_(ids)[0].tolist() == [0, 1, 2, 3] and np.allclose(np_(w)[0], 0.25)
    assert np_(ids)[1].tolist() == [3, 55, 17, 40]
    assert np_(ids)[2, 0] == 50 and np_(w)[2, 0] > 0.999999
    assert np_(ids)[3].tolist() == [0, 1, 2, 3]
    assert np.abs(np_(w) - tv).max() <= W_TOL


def test_route_topk_strided_rows_and_preallocated_out():
    """Logits rows with a leading stride (a slice of a wider buffer), outputs
    written into caller tensors."""
    M, n, k = 7, 128, 8
    wide = torch.from_numpy(_logits(M, 160, seed=77)).to(DEV)
    view = wide[:, 16:16 + n]
    ids = torch.empty((M, k), dtype=torch.int32, device=DEV)
    w = torch.empty((M, k), dtype=torch.float32, device=DEV)
    r = moe_layer.route_topk(view, k, out=(ids, w))
    torch.cuda.synchronize()
    assert r[0] is ids and r[1] is w
    ti, tv = ops.route_topk_np(np_(view), k)
    assert np.array_equal(np_(ids), ti)
    assert np.abs(np_(w) - tv).max() <= W_TOL


def _stack(dext, n_exp, H, Mi, seed):
    parts = {q: [] for q in ("gate_wp", "gate_ws", "up_wp", "up_ws", "down_wp", "down_ws")}
    for e in range(n_exp):
        for nm, (rows, cols), off in (("gate", (Mi, H), 0), ("up", (Mi, H), 1), ("down", (H, Mi), 2)):
            q, s = rand_weight(dext, rows, cols, seed + 3 * e + off)
            parts[nm + "_wp"].append(q)
            parts[nm + "_ws"].append(s)
    return moe_layer.StackedExperts(**{q: torch.stack(v).contiguous() for q, v in parts.items()})


def test_route_tables_drive_drop_in_ops(dext):
    """route_topk -> route_tables -> moe_gateup_tab / moe_down_tab / moe_combine
    gives the same bits as the host pointer lists built from the same ids
    (runtime/model_runner_v2.py:279-289)."""
    n_exp, H, Mi, M, k = 16, 512, 256, 3, 4
    stack = _stack(dext, n_exp, H, Mi, seed=3100)
    g = torch.Generator(device=DEV)
    g.manual_seed(8)
    x = torch.randn((M, H), generator=g, device=DEV).bfloat16()
    xq, xs = dext.prequant(x)
    logits = torch.randn((M, n_exp), generator=g, device=DEV)
    ids, w = moe_layer.route_topk(logits, k)
    gu_wp, gu_ws, dn_wp, dn_ws = moe_layer.route_tables(ids, stack)
    gu_d = dext.moe_gateup_tab(xq, xs, gu_wp, gu_ws, k, M, Mi, H)
    yd_d = dext.moe_down_tab(gu_d, dn_wp, dn_ws, k, M, H, Mi)
    out_d = dext.moe_combine(yd_d, w, M)
    torch.cuda.synchronize()
    flat = np_(ids).reshape(-1).tolist()
    gw, gs, dw, ds = [], [], [], []
    for m in range(M):
        row = flat[m * k:(m + 1) * k]
        gw += [stack.gate_wp[e] for e in row] + [stack.up_wp[e] for e in row]
        gs += [stack.gate_ws[e] for e in row] + [stack.up_ws[e] for e in row]
        dw += [stack.down_wp[e] for e in row]
        ds += [stack.down_ws[e] for e in row]
    ptr = np.array([t.data_ptr() for t in gw], np.int64)
    assert np.array_equal(np_(gu_wp), ptr)
    assert np.array_equal(np_(dn_ws), np.array([t.data_ptr() for t in ds], np.int64))
    gu_h = dext.moe_gateup(xq, xs, gw, gs, k, M, Mi, H)
    yd_h = dext.moe_down(gu_h, dw, ds, k, M, H, Mi)
    out_h = dext.moe_combine(yd_h, w, M)
    torch.cuda.synchronize()
    assert torch.equal(gu_d, gu_h) and torch.equal(yd_d, yd_h) and torch.equal(out_d, out_h)


def test_fused_layer_device_routing_in_graph(dext):
    """Per layer route_topk + the fused layer with device routing, 3 layers in
    one captured HIP graph; fresh logits are copied into the graph's input
    before each replay.  Every replay equals the eager chain with host-side
    routing from the oracle's ids and the device's weights."""
    n_exp, E, H, Mi, L = 16, 8, 2048, 768, 3
    stack = _stack(dext, n_exp, H, Mi, seed=4100)
    g = torch.Generator(device=DEV)
    g.manual_seed(12)
    x0 = torch.randn(H, generator=g, device=DEV).bfloat16()
    logits = torch.empty((L, n_exp), dtype=torch.float32, device=DEV)
    ids = [torch.empty(E, dtype=torch.int32, device=DEV) for _ in range(L)]
    ws = [torch.empty(E, dtype=torch.float32, device=DEV) for _ in range(L)]
    outs = [torch.empty(H, dtype=torch.float32, device=DEV) for _ in range(L)]
    bufs = [torch.empty(H, dtype=torch.bfloat16, device=DEV) for _ in range(L)]
    wsp = moe_layer.workspace(E, Mi, H)
    calls, src = [], x0
    for i in range(L):
        calls.append(moe_layer.DecodeLayerCall(src, ids[i], ws[i], stack, outs[i], bufs[i], wsp))
        src = bufs[i]

    def step():
        for i in range(L):
            moe_layer.route_topk(logits[i:i + 1], E, out=(ids[i].view(1, E), ws[i].view(1, E)))
            calls[i]()

    logits.copy_(torch.randn((L, n_exp), generator=g, device=DEV))
    step()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            step()
    torch.cuda.synchronize()
    hws = moe_layer.workspace(E, Mi, H)
    for rep in range(3):
        lg = torch.randn((L, n_exp), generator=g, device=DEV)
        logits.copy_(lg)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ti, _ = ops.route_topk_np(np_(lg), E)
        src = x0
        for i in range(L):
            assert np_(ids[i]).tolist() == ti[i].tolist(), (rep, i)
            o, r = moe_layer.decode_layer(src, ti[i].tolist(), np_(ws[i]).tolist(), stack,
                                          resid=torch.empty(H, dtype=torch.bfloat16, device=DEV), ws=hws)
            torch.cuda.synchronize()
            assert torch.equal(o, outs[i]) and torch.equal(r, bufs[i]), (rep, i)
            src = r
        log(f"  replay {rep}: device routing in the graph equals host routing")
    assert moe_layer.layer_status(wsp) == 0 and moe_layer.layer_status(hws) == 0


@pytest.mark.parametrize("n_exp,E,H,Mi,norm", [(128, 8, 2048, 768, True), (16, 8, 1024, 256, True),
                                               (200, 4, 512, 96, False), (9, 2, 512, 64, True)])
def test_fused_layer_routes_itself(dext, n_exp, E, H, Mi, norm):
    """mxfp4_moe_decode_layer_routed: the in-launch routing gives the oracle's
    ids, and the output equals the host-routed launch with those ids and the
    same weights, bit for bit."""
    stack = _stack(dext, n_exp, H, Mi, seed=5100 + n_exp)
    g = torch.Generator(device=DEV)
    g.manual_seed(n_exp + E)
    ws1, ws2 = moe_layer.workspace(E, Mi, H), moe_layer.workspace(E, Mi, H)
    for it in range(3):
        x = torch.randn((1, H), generator=g, device=DEV).bfloat16()
        lg = torch.randn(n_exp, generator=g, device=DEV) * 2
        r1 = torch.empty(H, dtype=torch.bfloat16, device=DEV)
        o1, _, ids, w = moe_layer.decode_layer_routed(x, lg, E, stack, norm=norm, resid=r1, ws=ws1,
                                                      want_routing=True)
        torch.cuda.synchronize()
        ti, tv = ops.route_topk_np(np_(lg)[None], E, renorm=norm)
        assert np_(ids).tolist() == ti[0].tolist()
        assert np.abs(np_(w) - tv[0]).max() <= W_TOL
        r2 = torch.empty(H, dtype=torch.bfloat16, device=DEV)
        o2, _ = moe_layer.decode_layer(x, ti[0].tolist(), np_(w).tolist(), stack, resid=r2, ws=ws2)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(r1, r2), it
    assert moe_layer.layer_status(ws1) == 0 and moe_layer.layer_status(ws2) == 0
    log(f"  routed layer n={n_exp} E={E} H={H} Mi={Mi}: ids exact, output equals host routing")


def test_fused_routed_layers_in_graph(dext):
    """Three self-routing layers in one captured graph, replayed with fresh
    logits copied in before each replay; every replay equals eager."""
    n_exp, E, H, Mi, L = 32, 8, 2048, 768, 3
    stack = _stack(dext, n_exp, H, Mi, seed=6100)
    g = torch.Generator(device=DEV)
    g.manual_seed(21)
    x0 = torch.randn(H, generator=g, device=DEV).bfloat16()
    logits = torch.empty((L, n_exp), dtype=torch.float32, device=DEV)
    outs = [torch.empty(H, dtype=torch.float32, device=DEV) for _ in range(L)]
    bufs = [torch.empty(H, dtype=torch.bfloat16, device=DEV) for _ in range(L)]
    ids = [torch.empty(E, dtype=torch.int32, device=DEV) for _ in range(L)]
    ws_ = [torch.empty(E, dtype=torch.float32, device=DEV) for _ in range(L)]
    wsp = moe_layer.workspace(E, Mi, H)
    calls, src = [], x0
    for i in range(L):
        calls.append(moe_layer.RoutedLayerCall(src, logits[i], E, stack, outs[i], bufs[i], wsp,
                                               ids_out=ids[i], w_out=ws_[i]))
        src = bufs[i]

    def step():
        for c in calls:
            c()

    logits.copy_(torch.randn((L, n_exp), generator=g, device=DEV))
    step()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            step()
    torch.cuda.synchronize()
    for rep in range(3):
        logits.copy_(torch.randn((L, n_exp), generator=g, device=DEV))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs] + [bufs[-1].clone()]
        got_ids = [i.clone() for i in ids]
        _ = torch.randn(1024, device=DEV).sum().item()   # unrelated eager work
        step()
        torch.cuda.synchronize()
        for i in range(L):
            assert torch.equal(got[i], outs[i]) and torch.equal(got_ids[i], ids[i]), (rep, i)
            assert np_(ids[i]).tolist() == ops.route_topk_np(np_(logits[i])[None], E)[0][0].tolist()
        assert torch.equal(got[-1], bufs[-1])
        log(f"  replay {rep}: self-routing layers equal eager")
    assert moe_layer.layer_status(wsp) == 0
