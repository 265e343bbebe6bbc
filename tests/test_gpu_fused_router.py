"""GPU parity of mxfp4_moe_decode_layer_fused_router: the post-attention
residual, RMSNorm and router projection inside the MoE launch.

Checked against the same step run as separate calls of this library:
  * x_out and y_out bit for bit against mxfp4_rmsnorm_lin_pq's residual and
    normed row (the same arithmetic, runtime/model_runner.py:20-25);
  * the logits against rmsnorm_lin_pq's router projection (the same MXFP4
    operands, another split of K over the waves: fp32 rounding only) and
    against the float64 oracle of the MXFP4 product;
  * ids / weights against mxfp4_route_topk on the launch's own logits, exact;
  * the MoE output bit for bit against mxfp4_moe_decode_layer on y_out with
    those ids and weights.
Several launches share one workspace, interleaved with plain fused-layer
launches, and a captured graph replays them."""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import _lib, moe_layer
from oracle import mxfp4 as fmt
from tests.gpu_helpers import DEV, log, np_, rand_weight
from tests.test_gpu_decode_layer import make_stack

pytestmark = pytest.mark.gpu
H, MI, E = 2048, 768, 8
EPS = 1e-6


def _inputs(g, scale_o=1.0):
    xa = torch.randn(H, generator=g, device=DEV).bfloat16()
    o = torch.randn(H, generator=g, device=DEV) * scale_o
    nw = (1.0 + 0.1 * torch.randn(H, generator=g, device=DEV)).bfloat16()
    return xa, o.contiguous(), nw


def _reference(lib, xa, o, nw, rwp, rws, n_exp, experts):
    """The separate calls: rmsnorm_lin_pq (residual, norm, router), then the
    fused layer on the normed row with the given routing."""
    xr = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    yr = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    yq = torch.empty(H // 2, dtype=torch.uint8, device=DEV)
    ys = torch.empty(H // 32, dtype=torch.uint8, device=DEV)
    lr = torch.empty(n_exp, dtype=torch.float32, device=DEV)
    _lib.check(lib.mxfp4_rmsnorm_lin_pq(xa.data_ptr(), o.data_ptr(), nw.data_ptr(), EPS, 1, H, xr.data_ptr(),
                                        yr.data_ptr(), yq.data_ptr(), ys.data_ptr(), rwp.data_ptr(), rws.data_ptr(),
                                        n_exp, lr.data_ptr(), None), "rmsnorm_lin_pq")
    return xr, yr, yq, ys, lr


@pytest.mark.parametrize("n_exp", [32, 128])
def test_fused_router_matches_separate_calls(dext, n_exp):
    lib = _lib.load()
    experts = make_stack(dext, n_exp, H, MI, seed=12000 + n_exp)
    rwp, rws = rand_weight(dext, n_exp, H, seed=12500 + n_exp, std=0.05)
    g = torch.Generator(device=DEV)
    g.manual_seed(n_exp)
    ws = moe_layer.workspace(E, MI, H)
    plain_out = torch.empty(H, dtype=torch.float32, device=DEV)
    for it in range(4):
        xa, o, nw = _inputs(g)
        outs = dict(out=torch.empty(H, dtype=torch.float32, device=DEV),
                    x_out=torch.empty(H, dtype=torch.bfloat16, device=DEV),
                    y_out=torch.empty(H, dtype=torch.bfloat16, device=DEV),
                    logits_out=torch.empty(n_exp, dtype=torch.float32, device=DEV),
                    ids_out=torch.empty(E, dtype=torch.int32, device=DEV),
                    w_out=torch.empty(E, dtype=torch.float32, device=DEV))
        call = moe_layer.FusedRouterLayerCall(xa, o, nw, EPS, rwp, rws, E, experts, outs["out"], ws,
                                              x_out=outs["x_out"], y_out=outs["y_out"],
                                              logits_out=outs["logits_out"], ids_out=outs["ids_out"],
                                              w_out=outs["w_out"])
        call()
        torch.cuda.synchronize()
        assert moe_layer.layer_status(ws) == 0
        xr, yr, yq, ys, lr = _reference(lib, xa, o, nw, rwp, rws, n_exp, experts)
        torch.cuda.synchronize()
        assert torch.equal(outs["x_out"], xr), "residual differs from rmsnorm_lin_pq"
        assert torch.equal(outs["y_out"], yr), "normed row differs from rmsnorm_lin_pq"
        lg, lref = np_(outs["logits_out"]).astype(np.float64), np_(lr).astype(np.float64)
        # float64 oracle of the MXFP4 product
        a = fmt.dequant_rows(np_(yq)[None], np_(ys)[None], H).astype(np.float64)
        wd = fmt.dequant_rows(np_(rwp), np_(rws), H).astype(np.float64)
        lor = (a @ wd.T)[0]
        span = np.abs(lor).max()
        d1, d2 = np.abs(lg - lref).max() / span, np.abs(lg - lor).max() / span
        log(f"  n_exp={n_exp} launch {it}: logits vs rmsnorm_lin_pq {d1:.2e}, vs oracle {d2:.2e}")
        assert d1 <= 1e-5 and d2 <= 1e-5
        ids, w = moe_layer.route_topk(outs["logits_out"][None], E)
        assert torch.equal(outs["ids_out"], ids[0]), "ids differ from route_topk on the launch's logits"
        assert torch.equal(outs["w_out"], w[0])
        ref = torch.empty(H, dtype=torch.float32, device=DEV)
        moe_layer.decode_layer(outs["y_out"], outs["ids_out"], outs["w_out"], experts, out=ref, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(outs["out"], ref), "MoE output differs from the fused layer on y_out"
        # a plain launch on the same workspace between fused ones keeps the launch counts in step
        moe_layer.decode_layer(outs["y_out"], [int(i) for i in ids[0].tolist()], [float(v) for v in w[0].tolist()],
                               experts, out=plain_out, ws=ws)
        torch.cuda.synchronize()
        assert moe_layer.layer_status(ws) == 0


def test_fused_router_graph_replays(dext):
    n_exp = 32
    experts = make_stack(dext, n_exp, H, MI, seed=13000)
    rwp, rws = rand_weight(dext, n_exp, H, seed=13100, std=0.05)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    xa, o, nw = _inputs(g)
    ws = moe_layer.workspace(E, MI, H)
    out = torch.empty(H, dtype=torch.float32, device=DEV)
    x_out = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    call = moe_layer.FusedRouterLayerCall(xa, o, nw, EPS, rwp, rws, E, experts, out, ws, x_out=x_out)
    call()
    torch.cuda.synchronize()
    eager = (out.clone(), x_out.clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            call()
            call()
    torch.cuda.synchronize()
    for rep in range(4):
        out.zero_()
        x_out.zero_()
        _ = torch.randn(1024, device=DEV).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]) and torch.equal(x_out, eager[1]), f"replay {rep}"
    assert moe_layer.layer_status(ws) == 0


def test_fused_router_argument_checks(dext):
    lib = _lib.load()
    p = 256
    args = [p, p, p, 1e-6, p, p, 1, None, None, None, None, None, p, p, p, p, p, p]
    ws = moe_layer.workspace(E, MI, H)
    tail = [ws.data_ptr(), ws.numel(), None]
    assert lib.mxfp4_moe_decode_layer_fused_router(*args, 40, E, H, MI, p, *tail) == -1
    assert "multiple of 16" in lib.mxfp4_last_error().decode()
    assert lib.mxfp4_moe_decode_layer_fused_router(*args, 32, E, 1024, MI, p, *tail) == -1
    assert "2048" in lib.mxfp4_last_error().decode()


def _qkv_reference(lib, x_out, out, qnw, qwp, qws, nq):
    """The next layer's input residual + norm + q|k|v as the separate
    mxfp4_rmsnorm_lin_pq call."""
    xn = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    qkv = torch.empty(nq, dtype=torch.float32, device=DEV)
    _lib.check(lib.mxfp4_rmsnorm_lin_pq(x_out.data_ptr(), out.data_ptr(), qnw.data_ptr(), EPS, 1, H, xn.data_ptr(),
                                        None, None, None, qwp.data_ptr(), qws.data_ptr(), nq, qkv.data_ptr(), None),
               "rmsnorm_lin_pq")
    return xn, qkv


@pytest.mark.parametrize("nq", [5120, 1000])
def test_fused_router_qkv_tail_matches_separate_calls(dext, nq):
    """mxfp4_moe_decode_layer_fused_router_qkv: the MoE part equals the
    launch without the tail, and qkv_out / x_next equal the next layer's
    mxfp4_rmsnorm_lin_pq on (x_out, out) bit for bit.  The tail splits K in
    four parts, as rmsnorm_lin_pq does for 4081..8192 rows, so the reference
    projects onto 5120 rows whose first nq are the tail's.  Launches with and
    without the tail, and plain fused-layer launches, share one workspace."""
    lib = _lib.load()
    n_exp = 128
    experts = make_stack(dext, n_exp, H, MI, seed=14000 + nq)
    rwp, rws = rand_weight(dext, n_exp, H, seed=14100 + nq, std=0.05)
    nref = 5120
    qwp_all, qws_all = rand_weight(dext, nref, H, seed=14200 + nq, std=0.05)
    qwp, qws = qwp_all[:nq], qws_all[:nq]
    g = torch.Generator(device=DEV)
    g.manual_seed(nq)
    ws = moe_layer.workspace(E, MI, H)
    for it in range(4):
        xa, o, _ = _inputs(g)
        nw = (1.0 + 0.1 * torch.randn(H, generator=g, device=DEV)).bfloat16()
        qnw = (1.0 + 0.1 * torch.randn(H, generator=g, device=DEV)).bfloat16()
        out = torch.empty(H, dtype=torch.float32, device=DEV)
        x_out = torch.empty(H, dtype=torch.bfloat16, device=DEV)
        qkv = torch.full((nq,), float("nan"), dtype=torch.float32, device=DEV)
        x_next = torch.empty(H, dtype=torch.bfloat16, device=DEV)
        ids_out = torch.empty(E, dtype=torch.int32, device=DEV)
        w_out = torch.empty(E, dtype=torch.float32, device=DEV)
        moe_layer.FusedRouterLayerCall(xa, o, nw, EPS, rwp, rws, E, experts, out, ws, x_out=x_out, ids_out=ids_out,
                                       w_out=w_out, next_qkv=(qnw, qwp, qws, qkv, x_next))()
        torch.cuda.synchronize()
        assert moe_layer.layer_status(ws) == 0
        # the same launch without the tail
        out2 = torch.empty(H, dtype=torch.float32, device=DEV)
        x_out2 = torch.empty(H, dtype=torch.bfloat16, device=DEV)
        moe_layer.FusedRouterLayerCall(xa, o, nw, EPS, rwp, rws, E, experts, out2, ws, x_out=x_out2)()
        xn_ref, qkv_ref = _qkv_reference(lib, x_out2, out2, qnw, qwp_all, qws_all, nref)
        qkv_ref = qkv_ref[:nq]
        torch.cuda.synchronize()
        assert moe_layer.layer_status(ws) == 0
        assert torch.equal(out, out2) and torch.equal(x_out, x_out2), "MoE part differs from the launch without tail"
        assert torch.equal(x_next, xn_ref), "x_next differs from rmsnorm_lin_pq's residual"
        if not torch.equal(qkv, qkv_ref):
            a, b = np_(qkv), np_(qkv_ref)
            bad = np.nonzero(a != b)[0]
            fin = np.isfinite(a)
            rel = np.abs(a[fin] - b[fin]) / (np.abs(b[fin]) + 1e-6)
            log(f"  nq={nq} launch {it}: {bad.size} of {nq} rows differ, first {bad[:12].tolist()}, "
                f"finite {int(fin.sum())}, median rel of finite {float(np.median(rel)) if rel.size else -1:.3e}, "
                f"bad by wave {np.bincount((bad % 64) // 16, minlength=4).tolist()}, by lane {np.bincount(bad % 16, minlength=16).tolist()}, "
                f"ratio a/b first {(a[bad[:6]] / b[bad[:6]]).tolist()}")
        assert torch.equal(qkv, qkv_ref), "q|k|v differs from rmsnorm_lin_pq"
        log(f"  nq={nq} launch {it}: out, x_next and q|k|v equal the separate calls "
            f"(|qkv| max {float(qkv.abs().max()):.3f})")
        # a plain launch in between keeps every launch count in step
        moe_layer.decode_layer(x_out, ids_out, w_out, experts, ws=ws)
        torch.cuda.synchronize()
        assert moe_layer.layer_status(ws) == 0


def test_fused_router_qkv_tail_graph_replays(dext):
    """Two chained tail launches (the second's x is the first's x_next) in a
    captured graph; every replay equals the eager run."""
    n_exp, nq = 32, 5120
    experts = make_stack(dext, n_exp, H, MI, seed=15000)
    rwp, rws = rand_weight(dext, n_exp, H, seed=15100, std=0.05)
    qwp, qws = rand_weight(dext, nq, H, seed=15200, std=0.05)
    g = torch.Generator(device=DEV)
    g.manual_seed(6)
    xa, o, nw = _inputs(g)
    ws = moe_layer.workspace(E, MI, H)
    out = torch.empty(H, dtype=torch.float32, device=DEV)
    x_out = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    x_next = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    x_next2 = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    qkv = torch.empty(nq, dtype=torch.float32, device=DEV)
    qkv2 = torch.empty(nq, dtype=torch.float32, device=DEV)
    calls = [moe_layer.FusedRouterLayerCall(xa, o, nw, EPS, rwp, rws, E, experts, out, ws, x_out=x_out,
                                            next_qkv=(nw, qwp, qws, qkv, x_next)),
             moe_layer.FusedRouterLayerCall(x_next, o, nw, EPS, rwp, rws, E, experts, out, ws, x_out=x_out,
                                            next_qkv=(nw, qwp, qws, qkv2, x_next2))]

    def run():
        for c in calls:
            c()

    run()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (qkv, qkv2, x_next2, out)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.synchronize()
    for rep in range(4):
        for t in (qkv, qkv2, x_next2, out):
            t.zero_()
        _ = torch.randn(1024, device=DEV).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip((qkv, qkv2, x_next2, out), eager)), f"replay {rep}"
    assert moe_layer.layer_status(ws) == 0


def test_fused_router_qkv_argument_checks(dext):
    lib = _lib.load()
    p = 256
    args = [p, p, p, 1e-6, p, p, 1, None, None, None, None, None, p, p, p, p, p, p, 32, E, H, MI]
    ws = moe_layer.workspace(E, MI, H)
    tail = [p, ws.data_ptr(), ws.numel(), None]
    assert lib.mxfp4_moe_decode_layer_fused_router_qkv(*args, p, p, p, 0, p, None, *tail) == -1
    assert "Nq=0" in lib.mxfp4_last_error().decode()
    assert lib.mxfp4_moe_decode_layer_fused_router_qkv(*args, p, p, p, 8193, p, None, *tail) == -1
    assert lib.mxfp4_moe_decode_layer_fused_router_qkv(*args, None, p, p, 64, p, None, *tail) == -1
    assert "null" in lib.mxfp4_last_error().decode()


@pytest.mark.parametrize("max_pos,pos", [(512, 300), (8192, 5000)])
def test_post_attn_matches_separate_calls(dext, max_pos, pos):
    """mxfp4_decode_layer_post_attn after mxfp4_attn_decode_fused_partials
    against the separate launches it replaces -- mxfp4_attn_decode_fused
    (chunk records + merge to MXFP4), mxfp4_lin_pq (o_proj), the fused
    router + MoE + q|k|v tail launch and the next layer's
    mxfp4_attn_decode_fused_partials -- bit for bit: the attention's MXFP4
    row, o_proj, residual, routing, MoE output, next q|k|v, x_next, the KV
    rows written in both layers and the next layer's chunk records.  Context
    5000 takes the merge's two-pass path (more than 64 chunks).  Three
    positions in a row on shared workspaces, with a plain fused-layer launch
    in between."""
    lib = _lib.load()
    Hq, Hkv, D, n_exp, nq = 32, 4, 128, 128, 5120
    experts = make_stack(dext, n_exp, H, MI, seed=16000 + pos)
    rwp, rws = rand_weight(dext, n_exp, H, seed=16100, std=0.05)
    owp, ows = rand_weight(dext, H, Hq * D, seed=16200, std=0.03)
    qwp, qws = rand_weight(dext, nq, H, seed=16300, std=0.05)
    g = torch.Generator(device=DEV)
    g.manual_seed(pos)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    qn2 = (1.0 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    kn2 = (1.0 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    qnw = (1.0 + 0.1 * torch.randn(H, generator=g, device=DEV)).bfloat16()
    r = torch.randint(0, 256, (max_pos, Hkv, D), generator=g, device=DEV, dtype=torch.int32)
    cache0 = ((r & 0x80) | (r & 0x3F)).to(torch.uint8)     # |v| < 2, no NaN code
    kv = {k: (cache0.clone(), cache0.flip(0).contiguous()) for k in ("sep", "fused")}
    kv2 = {k: (cache0.flip(1).contiguous(), cache0.flip(2).contiguous()) for k in kv}   # the next layer's
    nb = lib.mxfp4_attn_decode_workspace_size(1, Hq, max_pos)
    aws = {k: torch.empty((nb + 15) // 16 * 16, dtype=torch.uint8, device=DEV) for k in kv}
    aws2 = {k: torch.zeros((nb + 15) // 16 * 16, dtype=torch.uint8, device=DEV) for k in kv}
    lws = {k: moe_layer.workspace(E, MI, H) for k in kv}
    dpos = torch.zeros(1, dtype=torch.int32, device=DEV)
    s = torch.cuda.current_stream().cuda_stream

    def outs():
        return dict(aq=torch.empty(Hq * D // 2, dtype=torch.uint8, device=DEV),
                    as_=torch.empty(Hq * D // 32, dtype=torch.uint8, device=DEV),
                    oproj=torch.empty(H, dtype=torch.float32, device=DEV),
                    out=torch.empty(H, dtype=torch.float32, device=DEV),
                    x_out=torch.empty(H, dtype=torch.bfloat16, device=DEV),
                    ids=torch.empty(E, dtype=torch.int32, device=DEV),
                    w=torch.empty(E, dtype=torch.float32, device=DEV),
                    qkv=torch.empty(nq, dtype=torch.float32, device=DEV),
                    x_next=torch.empty(H, dtype=torch.bfloat16, device=DEV))

    for it, p in enumerate((pos, pos + 1, pos + 2)):
        dpos.fill_(p)
        qkv_in = (torch.randn(Hq * D + 2 * Hkv * D, generator=g, device=DEV) * 2.0).contiguous()
        xa = torch.randn(H, generator=g, device=DEV).bfloat16()
        nw = (1.0 + 0.1 * torch.randn(H, generator=g, device=DEV)).bfloat16()
        res = {}
        for mode in ("sep", "fused"):
            o = outs()
            kvk, kvv = kv[mode]
            common = (qkv_in.data_ptr(), qn.data_ptr(), kn.data_ptr(), EPS, 1e6, kvk.data_ptr(), kvv.data_ptr(),
                      dpos.data_ptr())
            if mode == "sep":
                _lib.check(lib.mxfp4_attn_decode_fused(*common, None, None, o["aq"].data_ptr(), o["as_"].data_ptr(), 1,
                                                       Hq, Hkv, D, max_pos, 0, aws[mode].data_ptr(), aws[mode].numel(),
                                                       s), "attn_decode_fused")
                _lib.check(lib.mxfp4_lin_pq(o["aq"].data_ptr(), o["as_"].data_ptr(), owp.data_ptr(), ows.data_ptr(),
                                            o["oproj"].data_ptr(), 1, H, Hq * D, Hq * D, s), "lin_pq")
                moe_layer.FusedRouterLayerCall(xa, o["oproj"], nw, EPS, rwp, rws, E, experts, o["out"], lws[mode],
                                               x_out=o["x_out"], ids_out=o["ids"], w_out=o["w"],
                                               next_qkv=(qnw, qwp, qws, o["qkv"], o["x_next"]))()
                _lib.check(lib.mxfp4_attn_decode_fused_partials(
                    o["qkv"].data_ptr(), qn2.data_ptr(), kn2.data_ptr(), EPS, 1e6, kv2[mode][0].data_ptr(),
                    kv2[mode][1].data_ptr(), dpos.data_ptr(), 1, Hq, Hkv, D, max_pos, 0, aws2[mode].data_ptr(),
                    aws2[mode].numel(), s), "attn_decode_fused_partials")
            else:
                _lib.check(lib.mxfp4_attn_decode_fused_partials(*common, 1, Hq, Hkv, D, max_pos, 0,
                                                                aws[mode].data_ptr(), aws[mode].numel(), s),
                           "attn_decode_fused_partials")
                moe_layer.PostAttnLayerCall(aws[mode], dpos, max_pos, owp, ows, o["oproj"], xa, nw, EPS, rwp, rws, E,
                                            experts, o["out"], lws[mode], aq_out=o["aq"], as_out=o["as_"],
                                            x_out=o["x_out"], ids_out=o["ids"], w_out=o["w"],
                                            next_qkv=(qnw, qwp, qws, o["qkv"], o["x_next"]),
                                            next_attn=(aws2[mode], kv2[mode][0], kv2[mode][1], qn2, kn2, Hkv, 1e6,
                                                       0))()
            torch.cuda.synchronize()
            assert moe_layer.layer_status(lws[mode]) == 0, mode
            res[mode] = o
        for k in res["sep"]:
            assert torch.equal(res["sep"][k], res["fused"][k]), f"position {p}: {k} differs from the separate launches"
        for a, b in zip(kv["sep"] + kv2["sep"], kv["fused"] + kv2["fused"]):
            assert torch.equal(a, b), f"position {p}: KV cache rows differ"
        # the next layer's chunk records (max, sum and the 128 column sums of
        # every chunk up to the position; the record's two pad floats are not written)
        nchunk = (max_pos + 63) // 64
        rec = {k: aws2[k][:Hq * nchunk * 132 * 4].view(torch.float32).view(Hq, nchunk, 132)[:, :p // 64 + 1]
               for k in kv}
        for sl in (slice(0, 2), slice(4, 132)):
            assert torch.equal(rec["sep"][..., sl], rec["fused"][..., sl]), f"position {p}: next layer's records differ"
        log(f"  max_pos={max_pos} position {p}: attention row, o_proj, MoE, routing, next q|k|v equal "
            f"(|oproj| max {float(res['fused']['oproj'].abs().max()):.3f})")
        # a plain launch on the fused workspace keeps the launch counts in step
        moe_layer.decode_layer(res["fused"]["x_out"], res["fused"]["ids"], res["fused"]["w"], experts, ws=lws["fused"])
        torch.cuda.synchronize()
        assert moe_layer.layer_status(lws["fused"]) == 0


def test_post_attn_argument_checks(dext):
    lib = _lib.load()
    p = 256
    ws = moe_layer.workspace(E, MI, H)
    nb = lib.mxfp4_attn_decode_workspace_size(1, 32, 512)
    head = [p, nb, p]
    mid = [p, p, p, p, p, 1e-6, p, p, 1, None, None, None, None, None, p, p, p, p, p, p, 128, E, H, MI,
           None, None, None, 0, None, None, None, 0, None, None, None, None, 0, 0.0, 0, p, ws.data_ptr(), ws.numel(),
           None]
    assert lib.mxfp4_decode_layer_post_attn(*head, 16, 512, None, None, *mid) == -1
    assert "Hq=16" in lib.mxfp4_last_error().decode()
    assert lib.mxfp4_decode_layer_post_attn(p, nb - 4, p, 32, 512, None, None, *mid) == -1
    assert "attention workspace" in lib.mxfp4_last_error().decode()
    assert lib.mxfp4_decode_layer_post_attn(*head, 32, 512, p, None, *mid) == -1
    assert "aq_out and as_out" in lib.mxfp4_last_error().decode()
    # the next layer's attention needs the q|k|v tail
    nxt = list(mid)
    nxt[30] = p
    nxt[31] = nb
    assert lib.mxfp4_decode_layer_post_attn(*head, 32, 512, None, None, *nxt) == -1
    assert "q|k|v tail" in lib.mxfp4_last_error().decode()
