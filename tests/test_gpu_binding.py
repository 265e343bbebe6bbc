"""The compiled torch binding (lib/mxfp4_ext.so) against the ctypes binding:
every op of the reference's two extension surfaces
(src/ext/mxfp4_binding.cpp:47-50, src/ext/mxfp4_decode_binding.cpp:232-243)
gives bit-identical outputs through both on the same inputs, and the
compiled ops launch on torch's current stream (a graph captured on a side
stream replays to the eager result).  Parity of the ops themselves with the
oracle is in the op tests, which run through the compiled binding."""
import numpy as np
import pytest
import torch

from tests.gpu_helpers import DEV, log, rand_weight

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def both():
    from moe_fused_inference_amd import get_decode_ext, get_ext
    return {b: (get_decode_ext(b), get_ext(b)) for b in ("compiled", "ctypes")}


def _run_all(d, l, inp):
    """Every op once; returns the outputs (KV caches written in place on copies)."""
    x, xw, ids, w, M, E, H, MI, kv = inp
    out = {}
    xq, xs = d.prequant(x)
    out["prequant"] = (xq, xs)
    out["lin_pq"] = d.lin_pq(xq, xs, xw[0], xw[1], M, xw[0].shape[0], H)
    out["forward"] = l.forward(x, xw[0], xw[1])
    out["forward_f16"] = l.forward(x.half(), xw[0], xw[1])
    gw = [ids[m][e]["gate"][0] for m in range(M) for e in range(E)] + \
         [ids[m][e]["up"][0] for m in range(M) for e in range(E)]
    gs = [ids[m][e]["gate"][1] for m in range(M) for e in range(E)] + \
         [ids[m][e]["up"][1] for m in range(M) for e in range(E)]
    dw = [ids[m][e]["down"][0] for m in range(M) for e in range(E)]
    ds = [ids[m][e]["down"][1] for m in range(M) for e in range(E)]
    gu = d.moe_gateup(xq, xs, gw, gs, E, M, MI, H)
    out["moe_gateup"] = gu
    yd = d.moe_down(gu, dw, ds, E, M, H, MI)
    out["moe_down"] = yd
    out["moe_combine"] = d.moe_combine(yd, w, M)

    def tab(ts):
        return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=DEV)
    out["moe_gateup_tab"] = d.moe_gateup_tab(xq, xs, tab(gw), tab(gs), E, M, MI, H)
    out["moe_down_tab"] = d.moe_down_tab(gu, tab(dw), tab(ds), E, M, H, MI)
    q, k, v, kvk0, kvv0, dpos = kv
    kvk, kvv = kvk0.clone(), kvv0.clone()
    d.kv_write(k, v, kvk, kvv, dpos, M)
    sc = torch.zeros((M, q.shape[1], kvk.shape[0]), dtype=torch.float32, device=DEV)
    out["attn_decode"] = d.attn_decode(q, kvk, kvv, dpos, sc, M)
    out["kv_write"] = (kvk, kvv)
    out["attn_scores"] = sc
    return out


def _inputs(d, M, E, H, MI, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = torch.randn((M, H), generator=g, device=DEV).bfloat16()
    xw = rand_weight(d, 320, H, seed + 1)
    pool = {}
    rng = np.random.default_rng(seed)
    ids = []
    for m in range(M):
        row = []
        for e in rng.choice(12, size=E, replace=False).tolist():
            if e not in pool:
                pool[e] = {"gate": rand_weight(d, MI, H, 1000 + 3 * e),
                           "up": rand_weight(d, MI, H, 1001 + 3 * e),
                           "down": rand_weight(d, H, MI, 1002 + 3 * e)}
            row.append(pool[e])
        ids.append(row)
    w = torch.softmax(torch.randn((M, E), generator=g, device=DEV), dim=1)
    Hq, Hkv, D, max_pos = 8, 2, 128, 256
    q = torch.randn((M, Hq, D), generator=g, device=DEV).bfloat16()
    k = torch.randn((M, Hkv, D), generator=g, device=DEV).bfloat16()
    v = torch.randn((M, Hkv, D), generator=g, device=DEV).bfloat16()
    kvk = torch.randint(0, 120, (max_pos, Hkv, D), generator=g, device=DEV, dtype=torch.uint8)
    kvv = torch.randint(0, 120, (max_pos, Hkv, D), generator=g, device=DEV, dtype=torch.uint8)
    dpos = torch.tensor([100], dtype=torch.int32, device=DEV)
    return x, xw, ids, w, M, E, H, MI, (q, k, v, kvk, kvv, dpos)


def _flat(o):
    return list(o) if isinstance(o, (tuple, list)) else [o]


@pytest.mark.parametrize("M,E,H,MI", [(1, 8, 2048, 768), (9, 8, 2048, 768), (3, 4, 320, 96)])
def test_bindings_bit_identical(both, M, E, H, MI):
    inp = _inputs(both["compiled"][0], M, E, H, MI, seed=M * 10 + E)
    res = {b: _run_all(*both[b], inp) for b in both}
    torch.cuda.synchronize()
    for op in res["compiled"]:
        a, b = _flat(res["compiled"][op]), _flat(res["ctypes"][op])
        for ta, tb in zip(a, b):
            assert ta.shape == tb.shape and ta.dtype == tb.dtype, op
            assert torch.equal(ta, tb), f"{op} differs between the bindings"
    log(f"  bindings bit-identical on {len(res['compiled'])} ops at M={M} E={E} H={H} Mi={MI}")


def test_compiled_ops_follow_the_current_stream(both):
    """prequant + moe_gateup + moe_down + moe_combine captured in a graph on a
    side stream (a launch on any other stream would break the capture) and
    replayed three times, each replay equal to the eager result."""
    d, _ = both["compiled"]
    M, E, H, MI = 1, 8, 2048, 768
    x, xw, ids, w, *_ = _inputs(d, M, E, H, MI, seed=3)
    gw = [r["gate"][0] for r in ids[0]] + [r["up"][0] for r in ids[0]]
    gs = [r["gate"][1] for r in ids[0]] + [r["up"][1] for r in ids[0]]
    dw = [r["down"][0] for r in ids[0]]
    ds = [r["down"][1] for r in ids[0]]

    def fn():
        xq, xs = d.prequant(x)
        gu = d.moe_gateup(xq, xs, gw, gs, E, M, MI, H)
        yd = d.moe_down(gu, dw, ds, E, M, H, MI)
        return d.moe_combine(yd, w, M)

    ref = fn().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            out = fn()
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
