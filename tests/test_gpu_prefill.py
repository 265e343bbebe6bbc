"""GPU parity of the grouped batched-token MoE (mxfp4_moe_group,
mxfp4_moe_prefill[_tab]), the counterpart of ModelRunnerV2.moe_compute
(runtime/model_runner_v2.py:108-122).

Oracle: oracle.ops.moe_prefill_ref -- the reference's per-expert loop on the
operands the op consumes (x -> fp16 -> MXFP4, fp32 silu(g)*u -> fp16 -> MXFP4,
bf16(y), bf16(y*score)), float64 accumulation.  The device sums a token's
slots in fp32 and rounds once to bf16, so the tolerance is the per-op cosine
plus a norm-wise max-rel that admits that last bf16 rounding (2^-9) and rare
E2M1 threshold flips of h (fp32 vs float64 g/u):
    cos >= 0.99999, max-rel <= 5e-3     (north star: 0.999 / 1e-2)
Tokens whose h sits within 1e-5 (relative) of an E2M1 threshold or an E8M0
scale boundary may round either way in any fp32 implementation; the oracle
flags them, the tight bound applies to the other tokens and the north-star
bound to all.  Routing bookkeeping is compared bit-exactly with a stable sort.
"""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import moe_layer
from oracle import ops
from tests.gpu_helpers import COS_NS, DEV, REL_NS, assert_close, log, np_, rand_weight

pytestmark = pytest.mark.gpu
COS_PF, REL_PF = 0.99999, 5e-3


def make_stack(dext, n_exp, H, Mi, seed):
    parts = {k: [] for k in ("gate_wp", "gate_ws", "up_wp", "up_ws", "down_wp", "down_ws")}
    for e in range(n_exp):
        for nm, (n, k), off in (("gate", (Mi, H), 0), ("up", (Mi, H), 1), ("down", (H, Mi), 2)):
            q, s = rand_weight(dext, n, k, seed + 3 * e + off)
            parts[nm + "_wp"].append(q)
            parts[nm + "_ws"].append(s)
    return moe_layer.StackedExperts(**{k: torch.stack(v).contiguous() for k, v in parts.items()})


def oracle_experts(stack, ids=None):
    ids = range(stack.n_experts) if ids is None else ids
    gw, gs, uw, us, dw, ds = (np_(getattr(stack, k)) for k in
                              ("gate_wp", "gate_ws", "up_wp", "up_ws", "down_wp", "down_ws"))
    return {e: ((gw[e], gs[e]), (uw[e], us[e]), (dw[e], ds[e])) for e in ids}


def check_prefill(out, x, ti, tv, experts, what):
    """Tight bound on tokens with a robust h quantization, north star on all."""
    T = x.shape[0]
    amb = np.zeros(T, bool)
    ref = ops.moe_prefill_ref(np_(x.float()), np_(ti), np_(tv.float()), experts, ambiguous=amb)
    y = np_(out.float()).astype(np.float64)
    assert_close(y, ref, COS_NS, REL_NS, what=what + " (all tokens, north star)")
    keep = ~amb
    log(f"  {what}: {int(amb.sum())} of {T} tokens with a threshold-adjacent h")
    if keep.any():
        # norm-wise max-rel over the kept tokens, relative to the whole output's max
        c = ops.cos_sim(y[keep], ref[keep])
        r = float(np.abs(y[keep] - ref[keep]).max() / np.abs(ref).max())
        log(f"  {what} (robust tokens): cos={c:.9f} max_rel={r:.3e}")
        assert c >= COS_PF and r <= REL_PF, (what, c, r)
    return ref


def route(g, T, n_exp, k, skew=False):
    logits = torch.randn((T, n_exp), generator=g, device=DEV)
    if skew:
        logits[:, 0] += 8.0     # nearly every token picks expert 0: several 128-token tiles
    p = torch.softmax(logits.float(), -1)
    tv, ti = torch.topk(p, k, dim=-1)
    tv = tv / tv.sum(-1, keepdim=True)
    return ti, tv.bfloat16()          # int64 ids, bf16 scores (runtime/model_runner_v2.py:100-106)


@pytest.mark.parametrize("T,k,n", [(333, 8, 128), (1000, 4, 6), (4096, 8, 130)])
def test_moe_group_matches_stable_sort(T, k, n):
    g = torch.Generator(device=DEV)
    g.manual_seed(1)
    topi = torch.randint(0, n, (T, k), generator=g, device=DEV)
    topi[5, 3] = -1
    topi[17, 0] = n + 7          # out of range: left out
    topi[30, 1] = n              # the ids next to the last expert match none
    topi[31, 2] = n + 1
    counts, offs, pairs = moe_layer.moe_group(topi, n)
    torch.cuda.synchronize()
    flat = np_(topi).reshape(-1)
    valid = (flat >= 0) & (flat < n)
    order = np.nonzero(valid)[0][np.argsort(flat[valid], kind="stable")]
    want_counts = np.bincount(flat[valid], minlength=n)
    want_offs = np.concatenate([[0], np.cumsum(want_counts)[:-1]])
    assert np.array_equal(np_(counts), want_counts)
    assert np.array_equal(np_(offs), want_offs)
    assert np.array_equal(np_(pairs)[:order.size], order)
    # the same bookkeeping as the oracle's grouping of the valid pairs
    experts, offsets, tok, slot = ops.group_by_expert(np.where(valid.reshape(T, k), np_(topi), n + 1000))
    assert np.array_equal((tok * k + slot)[:order.size], order)


@pytest.mark.parametrize("T,k,n_exp,H,Mi,skew", [
    (37, 4, 6, 512, 96, False),
    (1, 8, 12, 2048, 768, False),
    (300, 8, 16, 1024, 256, False),
    (260, 2, 4, 512, 160, True),
    (513, 4, 8, 256, 64, True),
    (700, 4, 8, 512, 512, True),
    (64, 4, 8, 640, 256, False),
])
def test_moe_compute_vs_oracle(dext, T, k, n_exp, H, Mi, skew):
    stack = make_stack(dext, n_exp, H, Mi, seed=70 + H + Mi)
    g = torch.Generator(device=DEV)
    g.manual_seed(T + n_exp)
    x = torch.randn((T, H), generator=g, device=DEV).bfloat16()
    ti, tv = route(g, T, n_exp, k, skew)
    out = moe_layer.moe_compute(x, ti, tv, stack)
    torch.cuda.synchronize()
    check_prefill(out, x, ti, tv, oracle_experts(stack), f"moe_compute T={T} k={k} n={n_exp} H={H} Mi={Mi}")
    if skew:
        log(f"  tokens on expert 0: {int((ti == 0).sum())}")


def test_moe_compute_invalid_ids_and_dict_form(dext):
    """The reference's dict of spec dicts (some experts absent) gives the
    same bits as the stacked form with the absent ids masked out."""
    n_exp, H, Mi, T, k = 8, 512, 128, 70, 4
    stack = make_stack(dext, n_exp, H, Mi, seed=400)
    g = torch.Generator(device=DEV)
    g.manual_seed(9)
    x = torch.randn((T, H), generator=g, device=DEV).bfloat16()
    ti, tv = route(g, T, n_exp, k)
    present = [0, 1, 2, 4, 5, 7]                        # experts 3 and 6 not loaded
    d = {e: stack.expert(e) for e in present}
    out_d = moe_layer.moe_compute(x, ti, tv, d)
    ti_masked = torch.where((ti == 3) | (ti == 6), torch.full_like(ti, -1), ti)
    out_s = moe_layer.moe_compute(x, ti_masked, tv, stack)
    torch.cuda.synchronize()
    assert torch.equal(out_d, out_s)
    check_prefill(out_d, x, ti, tv, oracle_experts(stack, present), "dict form, absent experts")


def test_moe_compute_workspace_reuse(dext):
    """One workspace serves consecutive calls of different sizes."""
    n_exp, H, Mi, k = 6, 512, 96, 4
    stack = make_stack(dext, n_exp, H, Mi, seed=800)
    ws = moe_layer.prefill_workspace(200, k, n_exp, H, Mi)
    g = torch.Generator(device=DEV)
    g.manual_seed(4)
    for T in (200, 31):
        x = torch.randn((T, H), generator=g, device=DEV).bfloat16()
        ti, tv = route(g, T, n_exp, k)
        out = moe_layer.moe_compute(x, ti, tv, stack, ws=ws)
        torch.cuda.synchronize()
        check_prefill(out, x, ti, tv, oracle_experts(stack), f"reuse T={T}")


def test_moe_compute_config3b_full_shape(dext):
    """Config 3b: 2048 tokens, top-8 of 128 experts, H=2048, Mi=768."""
    n_exp, H, Mi, T, k = 128, 2048, 768, 2048, 8
    stack = make_stack(dext, n_exp, H, Mi, seed=2000)
    g = torch.Generator(device=DEV)
    g.manual_seed(33)
    x = torch.randn((T, H), generator=g, device=DEV).bfloat16()
    ti, tv = route(g, T, n_exp, k)
    out = moe_layer.moe_compute(x, ti, tv, stack)
    torch.cuda.synchronize()
    log("  device done; oracle over 128 experts ...")
    check_prefill(out, x, ti, tv, oracle_experts(stack), "config 3b")
