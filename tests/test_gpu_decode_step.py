"""GPU parity of the whole decode step (moe_fused_inference_amd.decode_step)
and of its new ops, against oracle/step.py.

Tiny Qwen3-MoE-shaped model: 2 layers, H=2048, 4 query / 2 KV heads of 128,
8 experts top-4, Mi=256, vocab 512, cache of 256 positions with 100
positions of synthetic context.  Each step is compared layer by layer (the
residual stream after every layer) and on the logits; the token fed to the
next step is the GPU's own greedy token, so both sides stay on one path.
"""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import _lib
from moe_fused_inference_amd.decode_step import DecodeStep, ModelConfig, synthetic_model
from oracle import mxfp4 as fmt
from oracle import ops
from oracle import step as sref
from tests.gpu_helpers import DEV, assert_close, log, np_

pytestmark = pytest.mark.gpu

CFG = ModelConfig(n_layers=2, hidden=2048, n_heads=4, n_kv_heads=2, head_dim=128, n_experts=8, top_k=4,
                  moe_inter=256, vocab=512)
MAX_POS, CTX = 256, 100


def to_np(model, cfg):
    def pk(p):
        return (np_(p.wp), np_(p.ws))

    layers = []
    for lw in model.layers:
        ex = lw.experts
        experts = {e: tuple((np_(getattr(ex, p + "_wp")[e]), np_(getattr(ex, p + "_ws")[e])) for p in ("gate", "up", "down"))
                   for e in range(cfg.n_experts)}
        layers.append({"in_norm": np_(lw.in_norm.float()), "qkv": pk(lw.qkv), "q_norm": np_(lw.q_norm.float()),
                       "k_norm": np_(lw.k_norm.float()), "o": pk(lw.o), "post_norm": np_(lw.post_norm.float()),
                       "gate": pk(lw.gate), "experts": experts})
    return {"embed": pk(model.embed), "layers": layers, "final_norm": np_(model.final_norm.float()),
            "lm_head": pk(model.lm_head)}


@pytest.fixture(scope="module")
def tiny():
    model = synthetic_model(CFG, seed=11, device=DEV)
    torch.cuda.synchronize()
    return model, to_np(model, CFG)


def run_steps(model, wnp, M, n_steps, fused):
    st = DecodeStep(model, CFG, M=M, max_pos=MAX_POS, device=DEV)
    codec = st.kv_codec          # M = 1: kv_write's encoder (graph runner); M > 1: torch's (forward_batch)
    assert codec == (0 if M == 1 else 1)
    st.fill_cache(CTX, seed=5)
    ids = np.array([(37 * (i + 1)) % CFG.vocab for i in range(M)], np.int32)
    st.set_state(ids, CTX)
    torch.cuda.synchronize()
    kvk, kvv = np_(st.b.kvk).copy(), np_(st.b.kvv).copy()
    pos = CTX
    for step in range(n_steps):
        xs = []

        def hook(l, xa, moe):
            torch.cuda.synchronize()
            xs.append(np_((xa.float() + moe.bfloat16().float()).bfloat16().float()))

        st.run(on_layer=hook)
        torch.cuda.synchronize()
        logits = np_(st.b.logits)
        nxt = np_(st.b.ids)
        assert int(np_(st.b.dpos)[0]) == pos + M
        what = f"M={M} step {step} pos {pos}"
        # teacher-forced: every layer and the head start from the GPU's own
        # residual stream, so each is compared on identical inputs
        tf_logits, tf_xs = sref.step_ref(wnp, CFG, ids, pos, kvk.copy(), kvv.copy(), fused, x_teacher=xs,
                                         kv_codec=codec)
        for l in range(CFG.n_layers):
            assert_close(xs[l], tf_xs[l], 0.99999, 5e-3, what=f"{what} layer {l} residual (same input)")
        assert_close(logits, tf_logits, 0.9999, 1e-2, what=f"{what} logits (same input)")
        # free-running: the oracle's own chain end to end.  The final MXFP4
        # requantization of the normed residual turns a few bf16 flips of x
        # into whole-nibble (or whole-block scale) changes, so only cos is bound.
        ref_logits, ref_xs = sref.step_ref(wnp, CFG, ids, pos, kvk, kvv, fused, kv_codec=codec)
        for l in range(CFG.n_layers):
            assert_close(xs[l], ref_xs[l], 0.9999, 1e-2, what=f"{what} layer {l} residual (own chain)")
        assert_close(logits, ref_logits, 0.999, 1.0, what=f"{what} logits (own chain)")
        # greedy token = argmax of the GPU's own logits, exactly
        assert np.array_equal(nxt, sref.argmax_ref(logits)), what
        # the KV rows this step wrote: the reference codec on near-identical
        # inputs, so nearly every byte agrees
        gk, gv = np_(st.b.kvk), np_(st.b.kvv)
        rows = slice(pos, pos + M)
        agree = np.mean(gk[:, rows] == kvk[:, rows]), np.mean(gv[:, rows] == kvv[:, rows])
        assert min(agree) >= 0.98, f"{what}: KV bytes agree {agree}"
        log(f"  {what}: logits cos {ops.cos_sim(logits, ref_logits):.7f}, KV agreement {agree[0]:.4f}/{agree[1]:.4f}")
        # continue both sides with the GPU's caches and tokens
        kvk, kvv = gk.copy(), gv.copy()
        ids, pos = nxt.copy(), pos + M


def test_decode_step_one_token(tiny):
    model, wnp = tiny
    run_steps(model, wnp, 1, 3, fused=True)


def test_decode_step_batch(tiny):
    model, wnp = tiny
    run_steps(model, wnp, 4, 2, fused=False)


def test_decode_step_graph_replays_match_eager(tiny):
    """Steps replayed from a captured graph equal the same steps run eagerly."""
    model, _ = tiny
    outs = {}
    for mode in ("eager", "graph"):
        st = DecodeStep(model, CFG, M=1, max_pos=MAX_POS, device=DEV)
        st.fill_cache(CTX, seed=5)
        st.set_state([101], CTX)
        torch.cuda.synchronize()
        seq = []
        if mode == "eager":
            for _ in range(4):
                st.run()
                torch.cuda.synchronize()
                seq.append((np_(st.b.logits).copy(), int(np_(st.b.ids)[0])))
        else:
            graph = st.capture()          # runs step 1 eagerly while warming up
            torch.cuda.synchronize()
            seq.append((np_(st.b.logits).copy(), int(np_(st.b.ids)[0])))
            for _ in range(3):
                _ = torch.randn(1024, device=DEV).sum().item()   # unrelated eager work between replays
                graph.replay()
                torch.cuda.synchronize()
                seq.append((np_(st.b.logits).copy(), int(np_(st.b.ids)[0])))
        outs[mode] = seq
    for i, ((le, te), (lg, tg)) in enumerate(zip(outs["eager"], outs["graph"])):
        assert np.array_equal(le, lg) and te == tg, f"step {i}"


def test_embed_rows_exact(tiny):
    model, wnp = tiny
    lib = _lib.load()
    ids = torch.tensor([0, 5, 511, 77, 5], dtype=torch.int32, device=DEV)
    out = torch.empty((5, CFG.hidden), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.mxfp4_embed_rows(model.embed.wp.data_ptr(), model.embed.ws.data_ptr(), CFG.vocab, CFG.hidden,
                                    ids.data_ptr(), 5, out.data_ptr(), None), "embed_rows")
    torch.cuda.synchronize()
    ref = sref.embed_ref(*wnp["embed"], np_(ids), CFG.hidden)
    assert np.array_equal(np_(out.float()), ref)


@pytest.mark.parametrize("resid", [False, True])
def test_rmsnorm_quant(resid):
    """y matches rms_norm_ref up to rsqrt ulps, and yq/ys are exactly the
    quantizer's output on the y the kernel produced."""
    lib = _lib.load()
    g = torch.Generator(device=DEV)
    g.manual_seed(3 + resid)
    M, H = 5, 4096
    x = (torch.randn((M, H), generator=g, device=DEV) * 3).bfloat16()
    o = torch.randn((M, H), generator=g, device=DEV) if resid else None
    w = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).bfloat16()
    xo = torch.empty_like(x)
    y = torch.empty_like(x)
    yq = torch.empty((M, H // 2), dtype=torch.uint8, device=DEV)
    ys = torch.empty((M, H // 32), dtype=torch.uint8, device=DEV)
    _lib.check(lib.mxfp4_rmsnorm_quant(x.data_ptr(), o.data_ptr() if resid else None, w.data_ptr(), 1e-6, M, H,
                                       xo.data_ptr() if resid else None, y.data_ptr(), yq.data_ptr(), ys.data_ptr(),
                                       None), "rmsnorm_quant")
    torch.cuda.synchronize()
    xin = np_(x.float())
    if resid:
        want = fmt.bf16_round(xin + fmt.bf16_round(np_(o)))
        assert np.array_equal(np_(xo.float()), want)
        xin = want
    ref = sref.rms_norm_ref(xin, np_(w.float()), 1e-6)
    got = np_(y.float())
    ulp = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    assert np.mean(got == ref) >= 0.99 and ulp.max() <= 2 ** -7, (np.mean(got == ref), ulp.max())
    q, s = fmt.quantize_rows(got)
    assert np.array_equal(np_(yq), q) and np.array_equal(np_(ys), s)


@pytest.mark.parametrize("M,N,resid", [(1, 5120, False), (1, 128, True), (3, 2048, True), (8, 5120, True),
                                      (16, 20000, True), (5, 136, False)])
def test_rmsnorm_lin_pq_equals_the_two_calls(M, N, resid):
    """One launch of RMSNorm -> MXFP4 -> lin_pq gives exactly what
    mxfp4_rmsnorm_quant followed by mxfp4_lin_pq give: the residual, y, the
    MXFP4 rows and the projection, bit for bit (the same quantizer and the
    same split-K GEMV, A read from LDS instead of HBM)."""
    lib = _lib.load()
    g = torch.Generator(device=DEV)
    g.manual_seed(M * 1000 + N)
    H = 2048
    x = (torch.randn((M, H), generator=g, device=DEV) * 3).bfloat16()
    o = torch.randn((M, H), generator=g, device=DEV) if resid else None
    nw = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).bfloat16()
    w = (torch.randn((N, H), generator=g, device=DEV) * 0.02).bfloat16()
    wp = torch.empty((N, H // 2), dtype=torch.uint8, device=DEV)
    ws = torch.empty((N, H // 32), dtype=torch.uint8, device=DEV)
    _lib.check(lib.mxfp4_prequant(w.data_ptr(), H, N, H, H, wp.data_ptr(), ws.data_ptr(), None), "prequant")
    outs = []
    for fused in (False, True, "bare"):
        xo = torch.zeros_like(x)
        y = torch.zeros_like(x)
        yq = torch.zeros((M, H // 2), dtype=torch.uint8, device=DEV)
        ys = torch.zeros((M, H // 32), dtype=torch.uint8, device=DEV)
        out = torch.zeros((M, N), dtype=torch.float32, device=DEV)
        op = o.data_ptr() if resid else None
        xop = xo.data_ptr() if resid else None
        if fused:
            _lib.check(lib.mxfp4_rmsnorm_lin_pq(x.data_ptr(), op, nw.data_ptr(), 1e-6, M, H, xop, y.data_ptr(),
                                                yq.data_ptr(), ys.data_ptr(), wp.data_ptr(), ws.data_ptr(), N,
                                                out.data_ptr(), None), "rmsnorm_lin_pq")
        else:
            _lib.check(lib.mxfp4_rmsnorm_quant(x.data_ptr(), op, nw.data_ptr(), 1e-6, M, H, xop, y.data_ptr(),
                                               yq.data_ptr(), ys.data_ptr(), None), "rmsnorm_quant")
            _lib.check(lib.mxfp4_lin_pq(yq.data_ptr(), ys.data_ptr(), wp.data_ptr(), ws.data_ptr(), out.data_ptr(),
                                        M, N, H, H, None), "lin_pq")
        torch.cuda.synchronize()
        outs.append((xo, y, yq, ys, out))
    for name, a, b in zip(("x_out", "y", "yq", "ys", "out"), outs[0], outs[1]):
        assert torch.equal(a, b), f"M={M} N={N} resid={resid}: {name} differs"


@pytest.mark.parametrize("codec", [0, 1])
def test_qk_norm_rope_kv(codec):
    """Head RMSNorm + RoPE + KV write against oracle/step.py and the codecs
    of oracle/attn.py on the same fp32 projections: V bytes exactly the
    codec of bf16(v); q (bf16) and the K bytes up to the rsqrt / cos / sin
    ulps of fp32 (a bf16 flip moves a K byte by at most one code)."""
    from oracle import attn as aref
    lib = _lib.load()
    g = torch.Generator(device=DEV)
    g.manual_seed(21 + codec)
    M, Hq, Hkv, D, max_pos, base = 3, 8, 2, 128, 300, 290
    qkv = torch.randn((M, (Hq + 2 * Hkv) * D), generator=g, device=DEV) * 2
    qkv[0, (Hq + Hkv) * D:(Hq + Hkv) * D + 4] = torch.tensor([464.0, 470.0, 1.0625, 2.0 ** -8 * 3], device=DEV)
    qw = (1 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    kw = (1 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    dpos = torch.tensor([base], dtype=torch.int32, device=DEV)
    q_out = torch.zeros((M, Hq, D), dtype=torch.bfloat16, device=DEV)
    kvk = torch.zeros((max_pos, Hkv, D), dtype=torch.uint8, device=DEV)
    kvv = torch.zeros((max_pos, Hkv, D), dtype=torch.uint8, device=DEV)
    _lib.check(lib.mxfp4_qk_norm_rope_kv(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), 1e-6, 1e6, dpos.data_ptr(), M,
                                         Hq, Hkv, D, q_out.data_ptr(), kvk.data_ptr(), kvv.data_ptr(), max_pos, codec,
                                         None), "qk_norm_rope_kv")
    torch.cuda.synchronize()
    x = np_(qkv)
    pos = np.arange(base, base + M)
    q = sref.rope_ref(sref.rms_norm_ref(x[:, :Hq * D].reshape(M, Hq, D), np_(qw.float()), 1e-6, bf16_input=False),
                      pos, 1e6)
    k = sref.rope_ref(sref.rms_norm_ref(x[:, Hq * D:(Hq + Hkv) * D].reshape(M, Hkv, D), np_(kw.float()), 1e-6,
                                        bf16_input=False), pos, 1e6)
    v = fmt.bf16_round(x[:, (Hq + Hkv) * D:].reshape(M, Hkv, D))
    ck, cv = np.zeros((max_pos, Hkv, D), np.uint8), np.zeros((max_pos, Hkv, D), np.uint8)
    aref.kv_write_ref(k, v, ck, cv, base, codec)          # rows past max_pos are skipped on both sides
    assert np.array_equal(np_(kvv), cv)
    assert_close(np_(q_out.float()), q, 0.99999, 2e-2, what="q after norm + RoPE")
    gk = np_(kvk).astype(np.int64)
    assert np.mean(gk == ck) >= 0.995 and np.abs(gk - ck).max() <= 1
    if codec:
        assert np_(kvv)[base, 0, :4].tolist() == [0x7E, 0x7F, 0x38, 0x06]   # tie to 448, past it, tie, subnormal
    else:
        assert np_(kvv)[base, 0, :4].tolist() == [0x7F, 0x7F, 0x39, 0x01]   # saturation, half away from zero


def _argmax(lib, lg, ids, dpos, ws):
    _lib.check(lib.mxfp4_argmax_advance(lg.data_ptr(), lg.shape[0], lg.shape[1], ids.data_ptr(),
                                        dpos.data_ptr() if dpos is not None else None, ws.data_ptr(), ws.numel(),
                                        None), "argmax")
    torch.cuda.synchronize()


def test_argmax_first_maximum():
    lib = _lib.load()
    lg = torch.zeros((3, 1000), dtype=torch.float32, device=DEV)
    lg[0, 17] = 5.0
    lg[0, 900] = 5.0          # tie: the first index wins
    lg[1, :] = -1.0
    lg[1, 999] = 2.0
    lg[2, 3] = float("nan")   # NaN never wins
    lg[2, 4] = 1.0
    ids = torch.empty(3, dtype=torch.int32, device=DEV)
    dpos = torch.tensor([10], dtype=torch.int32, device=DEV)
    ws = torch.zeros(lib.mxfp4_argmax_workspace_size(3, 1000), dtype=torch.uint8, device=DEV)
    _argmax(lib, lg, ids, dpos, ws)
    assert ids.tolist() == [17, 999, 4] and int(dpos.item()) == 13
    assert int(ws[:16].count_nonzero()) == 0   # row counters back at zero


@pytest.mark.parametrize("V", [151936, 4097, 12289, 1003])
def test_argmax_slices_match_torch(V):
    """Rows spanning several workgroup slices (ties across slices, a row
    whose maximum is in the last partial slice, odd V on the scalar path),
    three calls in a row on one workspace, dpos advanced once per call."""
    lib = _lib.load()
    g = torch.Generator(device=DEV)
    g.manual_seed(V)
    M = 5
    lg = torch.randn((M, V), generator=g, device=DEV)
    lg[1, V // 3] = 50.0
    lg[1, V - 1] = 50.0               # tie across slices: the first wins
    lg[2, V - 1] = 60.0               # maximum at the very end
    lg[3, :] = float("nan")
    lg[3, V // 2] = -1.0              # one finite value among NaNs
    lg[4] = lg[4].round()             # many exact ties
    ws = torch.zeros(lib.mxfp4_argmax_workspace_size(M, V), dtype=torch.uint8, device=DEV)
    dpos = torch.tensor([7], dtype=torch.int32, device=DEV)
    ids = torch.empty(M, dtype=torch.int32, device=DEV)
    lgn = np_(lg)
    for call in range(3):
        _argmax(lib, lg, ids, dpos, ws)
        want = sref.argmax_ref(np.where(np.isnan(lgn), -np.inf, lgn))
        assert np.array_equal(np_(ids), want), (call, np_(ids), want)
        assert int(dpos.item()) == 7 + M * (call + 1)
    head = (M + 1) * 4
    assert int(ws[:head].count_nonzero()) == 0, "row counters not reset"


@pytest.mark.parametrize("M,Hq,Hkv,max_pos,base,codec", [
    (1, 32, 4, 4096, 4093, 0),    # the config-5 step: the new row in the last chunk
    (1, 32, 4, 4096, 64, 0),      # the new row first in its chunk
    (1, 8, 2, 300, 0, 1),         # empty context
    (3, 8, 2, 300, 62, 1),        # the step's rows straddle a chunk boundary
    (8, 32, 4, 1024, 700, 1),     # the batch step: two token groups per kv head
    (5, 16, 4, 200, 197, 0),      # rows past max_pos are not written
])
def test_attn_decode_fused_matches_two_ops(M, Hq, Hkv, max_pos, base, codec):
    """mxfp4_attn_decode_fused equals qk_norm_rope_kv followed by
    attn_decode_mx on the same projections and cache: the same cache bytes,
    raw scores, fp32 output and MXFP4 rows, bit for bit; and with sc and o
    NULL (how the step calls it) the same cache bytes and MXFP4 rows."""
    lib = _lib.load()
    g = torch.Generator(device=DEV)
    g.manual_seed(900 + M + base)
    D = 128
    qkv = torch.randn((M, (Hq + 2 * Hkv) * D), generator=g, device=DEV) * 2
    qw = (1 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    kw = (1 + 0.1 * torch.randn(D, generator=g, device=DEV)).bfloat16()
    dpos = torch.tensor([base], dtype=torch.int32, device=DEV)
    r = torch.randint(0, 256, (max_pos, Hkv, D), generator=g, device=DEV, dtype=torch.int32)
    cache = ((r & 0x80) | (r & 0x3F)).to(torch.uint8)        # |v| < 2, no NaN code
    wsb = lib.mxfp4_attn_decode_workspace_size(M, Hq, max_pos)
    outs = []
    for fused in (False, True, "bare"):
        kvk, kvv = cache.clone(), cache.flip(0).contiguous()
        sc = torch.zeros((M, Hq, max_pos), dtype=torch.float32, device=DEV)
        o = torch.zeros((M, Hq * D), dtype=torch.float32, device=DEV)
        oq = torch.zeros((M, Hq * D // 2), dtype=torch.uint8, device=DEV)
        os_ = torch.zeros((M, Hq * D // 32), dtype=torch.uint8, device=DEV)
        ws = torch.zeros(((wsb + 15) // 16 * 16,), dtype=torch.uint8, device=DEV)
        if fused:
            bare = fused == "bare"
            _lib.check(lib.mxfp4_attn_decode_fused(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), 1e-6, 1e6,
                                                   kvk.data_ptr(), kvv.data_ptr(), dpos.data_ptr(),
                                                   None if bare else sc.data_ptr(), None if bare else o.data_ptr(),
                                                   oq.data_ptr(), os_.data_ptr(), M, Hq, Hkv, D, max_pos,
                                                   codec, ws.data_ptr(), ws.numel(), None), "attn_decode_fused")
        else:
            q = torch.zeros((M, Hq, D), dtype=torch.bfloat16, device=DEV)
            _lib.check(lib.mxfp4_qk_norm_rope_kv(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), 1e-6, 1e6,
                                                 dpos.data_ptr(), M, Hq, Hkv, D, q.data_ptr(), kvk.data_ptr(),
                                                 kvv.data_ptr(), max_pos, codec, None), "qk_norm_rope_kv")
            _lib.check(lib.mxfp4_attn_decode_mx(q.data_ptr(), kvk.data_ptr(), kvv.data_ptr(), dpos.data_ptr(),
                                                sc.data_ptr(), o.data_ptr(), oq.data_ptr(), os_.data_ptr(), M, Hq, Hkv,
                                                D, max_pos, ws.data_ptr(), ws.numel(), None), "attn_decode_mx")
        torch.cuda.synchronize()
        outs.append((kvk, kvv, sc, o, oq, os_))
    live = torch.zeros((M, Hq, max_pos), dtype=torch.bool, device=DEV)
    for m in range(M):
        live[m, :, :min(base + m + 1, max_pos)] = True
    for name, a, b in zip(("kvk", "kvv", "sc", "o", "oq", "os"), outs[0], outs[1]):
        if name == "sc":
            a, b = a[live], b[live]
        assert torch.equal(a, b), f"M={M} base={base}: {name} differs"
    for name, a, b in zip(("kvk", "kvv", "sc", "o", "oq", "os"), outs[0], outs[2]):
        if name == "sc":
            assert not b.any(), "sc NULL: nothing written"
        elif name != "o":
            assert torch.equal(a, b), f"M={M} base={base}: {name} differs without sc / o"
    log(f"  M={M} Hq={Hq} base={base} codec={codec}: fused attention equal to the two launches")
