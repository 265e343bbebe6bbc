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
        tf_logits, tf_xs = sref.step_ref(wnp, CFG, ids, pos, kvk.copy(), kvv.copy(), fused, x_teacher=xs)
        for l in range(CFG.n_layers):
            assert_close(xs[l], tf_xs[l], 0.99999, 5e-3, what=f"{what} layer {l} residual (same input)")
        assert_close(logits, tf_logits, 0.9999, 1e-2, what=f"{what} logits (same input)")
        # free-running: the oracle's own chain end to end.  The final MXFP4
        # requantization of the normed residual turns a few bf16 flips of x
        # into whole-nibble (or whole-block scale) changes, so only cos is bound.
        ref_logits, ref_xs = sref.step_ref(wnp, CFG, ids, pos, kvk, kvv, fused)
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
    _lib.check(lib.mxfp4_argmax_advance(lg.data_ptr(), 3, 1000, ids.data_ptr(), dpos.data_ptr(), None), "argmax")
    torch.cuda.synchronize()
    assert ids.tolist() == [17, 999, 4] and int(dpos.item()) == 13
