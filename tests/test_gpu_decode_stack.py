"""GPU parity of the multi-layer decode launch (mxfp4_moe_decode_stack).

Two checks per case:
  * bit-exactness against the same layers run as chained one-layer launches
    (mxfp4_moe_decode_layer with device routing, x_{l+1} = its bf16 residual
    output): every layer's fp32 moe output y_l and bf16 x_{l+1};
  * every layer's y_l against the float64 dequant-to-BF16 oracle
    (oracle.ops.decode_layer_ref, runtime/model_runner.py:128-131) on that
    layer's own input x_l, to the north-star bound and a tighter one.
Repeated launches with different layer counts share one workspace, so the
buffer parity bookkeeping is exercised across launches.
"""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import moe_layer
from tests.gpu_helpers import COS_NS, DEV, REL_NS, assert_close, log, np_, pool_layer
from tests.test_gpu_decode_layer import make_stack, oracle_out, routing

pytestmark = pytest.mark.gpu
COS_TIGHT, REL_TIGHT = 0.99999, 2e-3


def stack_routes(g, n_exp, E, L):
    ids, ws = zip(*[routing(g, n_exp, E) for _ in range(L)])
    return torch.stack(ids).contiguous(), torch.stack(ws).contiguous()


def chained(x0, ids, w, layers, E):
    """The same layers as L one-layer launches; returns (x_all, y_all)."""
    H = layers[0].hidden
    lws = moe_layer.workspace(E, layers[0].inter, H)
    xs, ys = [], []
    src = x0
    for l, lay in enumerate(layers):
        out = torch.empty(H, dtype=torch.float32, device=DEV)
        resid = torch.empty(H, dtype=torch.bfloat16, device=DEV)
        moe_layer.decode_layer(src, ids[l].contiguous(), w[l].contiguous(), lay, out=out, resid=resid, ws=lws)
        xs.append(resid)
        ys.append(out)
        src = resid
    torch.cuda.synchronize()
    assert moe_layer.layer_status(lws) == 0
    return torch.stack(xs), torch.stack(ys)


@pytest.mark.parametrize("n_exp,E,H,Mi", [(12, 8, 2048, 768), (6, 4, 512, 256), (5, 3, 1024, 96),
                                          (4, 2, 1536, 160), (6, 4, 1024, 832), (3, 2, 512, 1024)])
def test_stack_matches_chained_layers_and_oracle(dext, n_exp, E, H, Mi):
    distinct = [make_stack(dext, n_exp, H, Mi, seed=7000 + 97 * i + H + Mi) for i in range(3)]
    g = torch.Generator(device=DEV)
    g.manual_seed(H * 3 + Mi)
    ws = moe_layer.stack_workspace(E, H, Mi)
    for it, (L, strict) in enumerate([(5, False), (1, False), (4, True), (2, False)]):
        layers = [distinct[(l + it) % 3] for l in range(L)]
        stack = moe_layer.LayerStack(layers)
        x0 = torch.randn(H, generator=g, device=DEV).bfloat16()
        ids, w = stack_routes(g, n_exp, E, L)
        log(f"stack n={n_exp} E={E} H={H} Mi={Mi} launch {it}: L={L} strict={strict}")
        x_out, x_all, y_all = moe_layer.decode_stack(x0, ids, w, stack, ws=ws, strict=strict, want_all=True)
        torch.cuda.synchronize()
        assert moe_layer.stack_status(ws) == 0
        cx, cy = chained(x0, ids, w, layers, E)
        assert torch.equal(y_all, cy), "moe outputs differ from chained one-layer launches"
        assert torch.equal(x_all, cx), "residual stream differs from chained one-layer launches"
        assert torch.equal(x_out, cx[-1])
        for l in range(L):
            xl = x0 if l == 0 else x_all[l - 1]
            ref = oracle_out(layers[l], xl, ids[l].tolist(), w[l].tolist())
            what = f"  layer {l}"
            assert_close(np_(y_all[l]), ref, COS_NS, REL_NS, what=what)
            assert_close(np_(y_all[l]), ref, COS_TIGHT, REL_TIGHT, what=what + " (tight)")


@pytest.mark.parametrize("L", [48, 131])
def test_stack_long_runs(dext, L):
    """A whole config-2 step (48 layers) and a run past the 128 layers whose
    routing and weight pointers the kernel stages in LDS (layers 128.. take the
    scalar-load path): bit-exact against chained one-layer launches, and the
    oracle on the first, a middle and the last layers.  Every layer has its
    own seeded weights, as in config 2 (a few stacks reused along the run
    amplify the residual stream layer after layer until it overflows)."""
    n_exp, E, H, Mi = 8, 8, 2048, 768
    layers = [make_stack(dext, n_exp, H, Mi, seed=9100 + 31 * l) for l in range(L)]
    stack = moe_layer.LayerStack(layers)
    g = torch.Generator(device=DEV)
    g.manual_seed(17 + L)
    x0 = torch.randn(H, generator=g, device=DEV).bfloat16()
    ids, w = stack_routes(g, n_exp, E, L)
    # beyond ~50 random layers the residual stream of this synthetic model
    # grows without bound (x reaches inf near layer 64 in both paths): damp
    # the long run's combine weights so every layer stays finite
    w = (w * (0.25 if L > 48 else 1.0)).contiguous()
    ws = moe_layer.stack_workspace(E, H, Mi)
    log(f"stack L={L}")
    x_out, x_all, y_all = moe_layer.decode_stack(x0, ids, w, stack, ws=ws, want_all=True)
    torch.cuda.synchronize()
    assert moe_layer.stack_status(ws) == 0
    cx, cy = chained(x0, ids, w, layers, E)
    assert torch.equal(y_all, cy), "moe outputs differ from chained one-layer launches"
    assert torch.equal(x_all, cx), "residual stream differs from chained one-layer launches"
    assert torch.equal(x_out, cx[-1])
    assert bool(torch.isfinite(y_all).all()), "non-finite moe output"
    for l in (0, L // 2, 127 if L > 128 else L - 2, L - 1):
        xl = x0 if l == 0 else x_all[l - 1]
        ref = oracle_out(layers[l], xl, ids[l].tolist(), w[l].tolist())
        assert_close(np_(y_all[l]), ref, COS_NS, REL_NS, what=f"  layer {l}")
        assert_close(np_(y_all[l]), ref, COS_TIGHT, REL_TIGHT, what=f"  layer {l} (tight)")


def test_stack_config2_expert_pool(dext):
    """Config 2 at its own shape: 48 layers, each with its own 128 seeded
    experts (15.4 GB resident), routing softmax -> top-8 -> renorm of fresh
    N(0, 1) logits per layer (runtime/model_runner_v2.py:189-192), so the ids
    span 0..127 as in the headline measurement.  The prefetching launch and the
    strict one equal chained one-layer launches bit for bit; layers 0, 23 and
    47 are checked against the float64 dequant-to-BF16 oracle."""
    n_exp, E, H, Mi, L = 128, 8, 2048, 768, 48
    layers = [pool_layer(dext, n_exp, H, Mi, seed=1000 + l) for l in range(L)]
    stack = moe_layer.LayerStack(layers)
    g = torch.Generator()
    g.manual_seed(2024)
    logits = torch.randn((L, n_exp), generator=g)
    tv, ti = torch.topk(torch.softmax(logits, -1), E, dim=-1)
    tv = tv / tv.sum(-1, keepdim=True)
    ids = ti.int().to(DEV).contiguous()
    w = tv.float().to(DEV).contiguous()
    used = torch.unique(ti)
    log(f"stack config 2: {L} layers x {n_exp} experts, {used.numel()} distinct ids in [{int(used.min())}, {int(used.max())}]")
    assert int(used.max()) >= 120 and used.numel() >= 100
    x0 = torch.randn(H, generator=g).bfloat16().to(DEV)
    ws = moe_layer.stack_workspace(E, H, Mi)
    cx, cy = chained(x0, ids, w, layers, E)
    for strict in (False, True):
        x_out, x_all, y_all = moe_layer.decode_stack(x0, ids, w, stack, ws=ws, strict=strict, want_all=True)
        torch.cuda.synchronize()
        assert moe_layer.stack_status(ws) == 0
        assert torch.equal(y_all, cy), f"strict={strict}: moe outputs differ from chained one-layer launches"
        assert torch.equal(x_all, cx), f"strict={strict}: residual stream differs from chained one-layer launches"
        assert torch.equal(x_out, cx[-1])
        log(f"  strict={strict}: 48 layers equal the chained launches bit for bit")
    assert bool(torch.isfinite(cy).all())
    for l in (0, 23, 47):
        xl = x0 if l == 0 else cx[l - 1]
        ref = oracle_out(layers[l], xl, ids[l].tolist(), w[l].tolist())
        assert_close(np_(cy[l]), ref, COS_NS, REL_NS, what=f"  layer {l}")
        assert_close(np_(cy[l]), ref, COS_TIGHT, REL_TIGHT, what=f"  layer {l} (tight)")
    del layers, stack
    torch.cuda.empty_cache()


def test_stack_strict_equals_prefetch(dext):
    n_exp, E, H, Mi = 10, 8, 2048, 768
    layers = [make_stack(dext, n_exp, H, Mi, seed=8100 + i) for i in range(2)] * 3
    stack = moe_layer.LayerStack(layers)
    g = torch.Generator(device=DEV)
    g.manual_seed(11)
    x0 = torch.randn(H, generator=g, device=DEV).bfloat16()
    ids, w = stack_routes(g, n_exp, E, len(layers))
    ws = moe_layer.stack_workspace(E, H, Mi)
    a = moe_layer.decode_stack(x0, ids, w, stack, ws=ws, strict=False, want_all=True)
    b = moe_layer.decode_stack(x0, ids, w, stack, ws=ws, strict=True, want_all=True)
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    assert moe_layer.stack_status(ws) == 0


def test_stack_graph_replays_match_eager(dext):
    """Two stack launches (x chained through both) captured in a HIP graph and
    replayed with eager work between replays; every replay equals eager."""
    n_exp, E, H, Mi = 10, 8, 2048, 768
    layers = [make_stack(dext, n_exp, H, Mi, seed=8300 + i) for i in range(3)]
    stack = moe_layer.LayerStack(layers)
    g = torch.Generator(device=DEV)
    g.manual_seed(13)
    x0 = torch.randn(H, generator=g, device=DEV).bfloat16()
    r1 = stack_routes(g, n_exp, E, 3)
    r2 = stack_routes(g, n_exp, E, 3)
    ws = moe_layer.stack_workspace(E, H, Mi)
    x1 = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    x2 = torch.empty(H, dtype=torch.bfloat16, device=DEV)
    y2 = torch.empty((3, H), dtype=torch.float32, device=DEV)
    calls = [moe_layer.DecodeStackCall(x0, r1[0], r1[1], stack, x1, ws),
             moe_layer.DecodeStackCall(x1, r2[0], r2[1], stack, x2, ws, y_all=y2)]

    def run():
        for c in calls:
            c()

    run()
    torch.cuda.synchronize()
    eager = (x2.clone(), y2.clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        run()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.synchronize()
    for rep in range(4):
        x2.zero_()
        y2.zero_()
        _ = torch.randn(1024, device=DEV).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(x2, eager[0]) and torch.equal(y2, eager[1]), f"replay {rep}, error flag {moe_layer.stack_status(ws)}"
        log(f"  replay {rep} matches eager")
    assert moe_layer.stack_status(ws) == 0


def test_stack_rejects_bad_arguments(dext):
    n_exp, E, H, Mi = 4, 2, 512, 64
    lay = make_stack(dext, n_exp, H, Mi, seed=8500)
    stack = moe_layer.LayerStack([lay, lay])
    x0 = torch.zeros(H, dtype=torch.bfloat16, device=DEV)
    ids = torch.zeros((2, E), dtype=torch.int32, device=DEV)
    w = torch.zeros((2, E), dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError):
        moe_layer.decode_stack(x0, ids[:1].contiguous(), w[:1].contiguous(), stack)   # L mismatch
    with pytest.raises(RuntimeError):
        moe_layer.decode_stack(x0, ids.long(), w, stack)
    with pytest.raises(RuntimeError):
        moe_layer.LayerStack([lay, make_stack(dext, n_exp, H, 96, seed=8501)])   # shapes differ
    # Mi above 1024: more g/u rows than the 32 workgroups of an XCD hold in registers
    big = make_stack(dext, 2, 512, 1056, seed=8502)
    with pytest.raises(RuntimeError, match="Mi=1056"):
        moe_layer.decode_stack(torch.zeros(512, dtype=torch.bfloat16, device=DEV),
                               torch.zeros((1, 2), dtype=torch.int32, device=DEV),
                               torch.zeros((1, 2), dtype=torch.float32, device=DEV), moe_layer.LayerStack([big]))
