"""GPU parity of the fused one-launch decode MoE layer (mxfp4_moe_decode_layer).

Oracle: the reference's dequant-to-BF16 expert path (runtime/model_runner.py:
128-131, dequant runtime/weight_store.py:27-44) on the UN-quantized bf16 x,
computed in float64 (oracle.ops.decode_layer_ref).  North-star tolerance:
cos >= 0.999 and norm-wise max-rel <= 1e-2; the kernel is expected to be far
inside it (E4M3 three-term activations, fp32 accumulation), so a tighter
bound is asserted as well.
"""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import moe_layer
from oracle import ops
from tests.gpu_helpers import COS_NS, DEV, REL_NS, assert_close, log, np_, rand_weight

pytestmark = pytest.mark.gpu
COS_TIGHT, REL_TIGHT = 0.99999, 2e-3


def make_stack(dext, n_exp, H, Mi, seed):
    parts = {k: [] for k in ("gate_wp", "gate_ws", "up_wp", "up_ws", "down_wp", "down_ws")}
    for e in range(n_exp):
        for nm, (n, k), off in (("gate", (Mi, H), 0), ("up", (Mi, H), 1), ("down", (H, Mi), 2)):
            q, s = rand_weight(dext, n, k, seed + 3 * e + off)
            parts[nm + "_wp"].append(q)
            parts[nm + "_ws"].append(s)
    return moe_layer.StackedExperts(**{k: torch.stack(v).contiguous() for k, v in parts.items()})


def oracle_out(stack, x, ids, w):
    experts = {}
    for e in set(int(i) for i in ids):
        experts[e] = tuple((np_(getattr(stack, p + "_wp")[e]), np_(getattr(stack, p + "_ws")[e]))
                           for p in ("gate", "up", "down"))
    return ops.decode_layer_ref(np_(x.float()).reshape(1, -1), np.array([ids]), np.array([w]), experts)[0]


def routing(g, n_exp, E):
    logits = torch.randn(n_exp, generator=g, device=DEV)
    p = torch.softmax(logits.float(), -1)
    tv, ti = torch.topk(p, E)
    tv = tv / tv.sum()
    return ti.int(), tv.float()


@pytest.mark.parametrize("n_exp,E,H,Mi", [(16, 8, 2048, 768), (6, 4, 512, 256), (5, 3, 1024, 96), (4, 2, 1536, 160)])
def test_decode_layer_vs_bf16_oracle(dext, n_exp, E, H, Mi):
    stack = make_stack(dext, n_exp, H, Mi, seed=500 + H)
    g = torch.Generator(device=DEV)
    g.manual_seed(H + Mi)
    ws = moe_layer.workspace(E, Mi, H)
    for it in range(3):  # repeated launches on one workspace: counters reset themselves
        x = torch.randn((1, H), generator=g, device=DEV).bfloat16()
        ti, tv = routing(g, n_exp, E)
        resid = torch.empty(H, dtype=torch.bfloat16, device=DEV)
        out, _ = moe_layer.decode_layer(x, ti.tolist(), tv.tolist(), stack, resid=resid, ws=ws)
        torch.cuda.synchronize()
        ref = oracle_out(stack, x, ti.tolist(), tv.tolist())
        assert_close(np_(out), ref, COS_NS, REL_NS, what=f"decode_layer n={n_exp} E={E} H={H} Mi={Mi} it={it}")
        assert_close(np_(out), ref, COS_TIGHT, REL_TIGHT, what="  (tight)")
        # residual: bf16(x + bf16(out)) exactly as runtime/model_runner_v2.py:208
        want = (x.reshape(-1).float() + out.bfloat16().float()).bfloat16()
        assert torch.equal(resid, want)
    assert moe_layer.layer_status(ws) == 0


def test_device_routing_equals_host_routing(dext):
    n_exp, E, H, Mi = 12, 8, 2048, 768
    stack = make_stack(dext, n_exp, H, Mi, seed=900)
    g = torch.Generator(device=DEV)
    g.manual_seed(3)
    x = torch.randn((1, H), generator=g, device=DEV).bfloat16()
    ti, tv = routing(g, n_exp, E)
    ws = moe_layer.workspace(E, Mi, H)
    o1, _ = moe_layer.decode_layer(x, ti.tolist(), tv.tolist(), stack, ws=ws)
    o2, _ = moe_layer.decode_layer(x, ti.contiguous(), tv.contiguous(), stack, ws=ws)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert moe_layer.layer_status(ws) == 0


def test_graph_replays_match_eager(dext):
    """A chain of 4 layers captured in a HIP graph, replayed several times with
    eager work and synchronisation in between; every replay equals eager."""
    n_exp, E, H, Mi = 10, 8, 2048, 768
    stack = make_stack(dext, n_exp, H, Mi, seed=1300)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    x0 = torch.randn(H, generator=g, device=DEV).bfloat16()
    routes = [routing(g, n_exp, E) for _ in range(4)]
    ws = moe_layer.workspace(E, Mi, H)
    bufs = [torch.empty(H, dtype=torch.bfloat16, device=DEV) for _ in range(4)]
    outs = [torch.empty(H, dtype=torch.float32, device=DEV) for _ in range(4)]
    calls = []
    src = x0
    for L in range(4):
        ti, tv = routes[L]
        calls.append(moe_layer.DecodeLayerCall(src, ti.tolist(), tv.tolist(), stack, outs[L], bufs[L], ws))
        src = bufs[L]

    def run():
        for c in calls:
            c()

    run()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs] + [bufs[-1].clone()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        run()  # warm on the side stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.synchronize()
    for rep in range(4):
        for o in outs:
            o.zero_()
        _ = torch.randn(1024, device=DEV).sum().item()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        for L in range(4):
            assert torch.equal(outs[L], eager[L]), (rep, L)
        assert torch.equal(bufs[-1], eager[-1])
        log(f"  replay {rep} matches eager")
    assert moe_layer.layer_status(ws) == 0
