"""Pins the per-operator CPU references (oracle/ops.py) on tiny inputs.

Each check reduces to something the mathematics fixes independently of the
oracle's code: explicit triple loops, one-hot / identity-like weights whose
product is a column selection, all-zero blocks, the combine's cap at 8 slots
(src/ext/mxfp4_decode.cu:296), the token-major table order
(runtime/model_runner_v2.py:279-286) and brute-force routing/grouping.
"""
import numpy as np
import pytest

from oracle import mxfp4 as fmt
from oracle import ops


def _q(x, kp=None):
    return fmt.quantize_rows(np.asarray(x, np.float32), kp=kp)


def test_lin_pq_ref_matches_explicit_loops():
    rng = np.random.default_rng(0)
    M, N, K = 3, 5, 70
    xq, xs = _q(rng.standard_normal((M, K)))
    wq, ws = _q(rng.standard_normal((N, K)))
    A = fmt.dequant_rows(xq, xs)
    W = fmt.dequant_rows(wq, ws)
    y = ops.lin_pq_ref(xq, xs, wq, ws)
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(A.shape[1]):
                s += float(A[m, k]) * float(W[n, k])
            assert abs(y[m, n] - s) <= 1e-12 * max(1.0, abs(s))


def test_lin_pq_ref_one_hot_weights_select_columns():
    # W[n] = one-hot at column perm[n] with value 1.0 -> y[:, n] = A[:, perm[n]]
    rng = np.random.default_rng(1)
    M, K = 4, 96
    perm = rng.permutation(K)[:16]
    W = np.zeros((16, K), np.float32)
    W[np.arange(16), perm] = 1.0
    wq, ws = _q(W)
    xq, xs = _q(rng.standard_normal((M, K)))
    y = ops.lin_pq_ref(xq, xs, wq, ws)
    A = fmt.dequant_rows(xq, xs)
    assert np.array_equal(y, A[:, perm].astype(np.float64))


def test_forward_ref_rounds_to_fp16_first():
    # 1 + 2^-12 is a bf16/fp32 value that fp16 rounds to 1.0: the block then
    # quantizes exactly as a block of 1.0 (src/ext/mxfp4_binding.cpp:31)
    x = np.full((1, 32), 1.0 + 2.0 ** -12, np.float32)
    xq, xs = ops.forward_act_quant_ref(x, 32)
    xq1, xs1 = _q(np.ones((1, 32)))
    assert np.array_equal(xq, xq1) and np.array_equal(xs, xs1)
    # values beyond the fp16 range become inf -> the reference's half cast
    assert np.isinf(fmt.f16_round(np.float32(70000.0)))


def test_zero_blocks_give_zero_output():
    wq, ws = _q(np.zeros((8, 64)))
    assert (ws == 127).all() and not wq.any()
    xq, xs = _q(np.ones((2, 64)))
    assert not ops.lin_pq_ref(xq, xs, wq, ws).any()


def _experts(rng, n_exp, N, K, scale=0.1):
    ws = []
    for _ in range(n_exp):
        ws.append(_q(rng.standard_normal((N, K)) * scale))
    return ws


def test_moe_gateup_ref_token_major_table():
    """Entry t = m*2E + proj*E + e lands in gu[m*E+e, proj*N:(proj+1)*N]."""
    rng = np.random.default_rng(2)
    E, M, N, K = 3, 2, 16, 64
    xq, xs = _q(rng.standard_normal((M, K)))
    table = _experts(rng, 2 * E * M, N, K)
    gu = ops.moe_gateup_ref(xq, xs, [t[0] for t in table], [t[1] for t in table], E, M, N)
    A = fmt.dequant_rows(xq, xs).astype(np.float64)
    for m in range(M):
        for proj in range(2):
            for e in range(E):
                W = fmt.dequant_rows(*table[m * 2 * E + proj * E + e]).astype(np.float64)
                assert np.allclose(gu[m * E + e, proj * N:(proj + 1) * N], W @ A[m], rtol=0, atol=1e-12)


def test_moe_down_ref_matches_manual_chain():
    rng = np.random.default_rng(3)
    E, M, N, K = 2, 2, 32, 96
    gu = rng.standard_normal((M * E, 2 * K)).astype(np.float32)
    table = _experts(rng, E * M, N, K)
    yd = ops.moe_down_ref(gu, [t[0] for t in table], [t[1] for t in table], E, M, N, K)
    for z in range(M * E):
        g, u = gu[z, :K].astype(np.float64), gu[z, K:].astype(np.float64)
        h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
        hq, hs = _q(h[None])
        W = fmt.dequant_rows(*table[z]).astype(np.float64)
        want = W @ fmt.dequant_rows(hq, hs)[0].astype(np.float64)
        # h differs from the fp32 chain by at most a few ulps -> compare loosely
        assert ops.cos_sim(yd[z], want) > 0.999


def test_moe_combine_ref_caps_at_eight_slots():
    rng = np.random.default_rng(4)
    M, E, N = 2, 9, 8
    yd = rng.standard_normal((M * E, N)).astype(np.float32)
    w = rng.random((M, E)).astype(np.float32)
    out = ops.moe_combine_ref(yd, w, M)
    for m in range(M):
        want = sum(np.float64(w[m, e]) * yd[m * E + e] for e in range(8))  # slot 8 ignored
        assert np.allclose(out[m], want, rtol=1e-6, atol=1e-6)
    # a single expert with weight 1 reproduces its row exactly
    one = ops.moe_combine_ref(yd[:1], np.ones((1, 1), np.float32), 1)
    assert np.array_equal(one[0], yd[0])


def _gapped_logits(rng, T, n, gap=1e-3):
    base = rng.permutation(n)[None, :].repeat(T, 0).astype(np.float64)
    for t in range(T):
        base[t] = rng.permutation(n)
    return (base * gap * 10 + rng.standard_normal((T, 1))).astype(np.float32)


def test_routing_indices_bruteforce():
    rng = np.random.default_rng(5)
    lg = _gapped_logits(rng, 9, 128)
    topi, topv = ops.route_ref(lg, k=8)
    assert np.array_equal(topi, ops.route_bruteforce(lg, k=8))
    assert np.allclose(topv.sum(-1), 1.0, atol=1e-6)
    assert (np.diff(topv, axis=-1) <= 0).all()


def test_group_by_expert_bruteforce():
    rng = np.random.default_rng(6)
    topi = rng.integers(0, 20, size=(9, 8))
    experts, offs, tok, slot = ops.group_by_expert(topi)
    assert list(experts) == sorted(set(topi.reshape(-1).tolist()))
    for g, e in enumerate(experts):
        pairs = [(t, s) for t in range(9) for s in range(8) if topi[t, s] == e]
        got = list(zip(tok[offs[g]:offs[g + 1]], slot[offs[g]:offs[g + 1]]))
        assert got == pairs
    assert offs[-1] == topi.size


def test_token_major_tables_order():
    topi = np.array([[3, 1], [1, 7]])
    gu, dn = ops.token_major_tables(topi, 2, 2)
    assert gu.tolist() == [6, 2, 7, 3, 2, 14, 3, 15]  # expert*2+proj
    assert dn.tolist() == [3, 1, 1, 7]


def test_decode_layer_ref_matches_per_expert_loop():
    rng = np.random.default_rng(7)
    H, Mi = 64, 32
    experts = {e: (_q(rng.standard_normal((Mi, H)) * 0.2), _q(rng.standard_normal((Mi, H)) * 0.2),
                   _q(rng.standard_normal((H, Mi)) * 0.2)) for e in range(4)}
    x = fmt.bf16_round(rng.standard_normal((1, H)).astype(np.float32))
    topi = np.array([[2, 0]])
    topv = np.array([[0.7, 0.3]], np.float32)
    out = ops.decode_layer_ref(x, topi, topv, experts)
    want = np.zeros(H)
    for s, e in enumerate(topi[0]):
        wg, wu, wd = (fmt.dequant_rows(*experts[e][j]).astype(np.float64) for j in range(3))
        g, u = wg @ x[0], wu @ x[0]
        want += topv[0, s] * (wd @ (g / (1 + np.exp(-g)) * u))
    assert np.allclose(out[0], want, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("M", [1, 3])
def test_cpu_baseline_close_to_fp32_oracle(M):
    """The dequant+BF16 chain (the timed CPU baseline) is within bf16 noise of
    the float64 oracle -- a sanity check of the baseline's semantics."""
    import torch
    rng = np.random.default_rng(8)
    H, Mi = 128, 64
    experts = {e: (_q(rng.standard_normal((Mi, H)) * 0.1), _q(rng.standard_normal((Mi, H)) * 0.1),
                   _q(rng.standard_normal((H, Mi)) * 0.1)) for e in range(6)}
    x = fmt.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    topi = np.stack([rng.permutation(6)[:4] for _ in range(M)])
    topv = rng.random((M, 4)).astype(np.float32)
    topv /= topv.sum(-1, keepdims=True)
    ref = ops.decode_layer_ref(x, topi, topv, experts)
    got = ops.dequant_bf16_moe_layer_torch(torch.from_numpy(x).bfloat16(), topi, topv, experts=experts)
    assert ops.cos_sim(got.float().numpy(), ref) > 0.995


def _rand_experts(rng, ids, H, Mi):
    ex = {}
    for e in ids:
        parts = []
        for n, k in ((Mi, H), (Mi, H), (H, Mi)):
            parts.append(fmt.quantize_rows((rng.standard_normal((n, k)) * 0.05).astype(np.float32)))
        ex[e] = tuple(parts)
    return ex


@pytest.mark.parametrize("skew", [False, True])
def test_moe_prefill_ref_matches_tokenwise_loop(skew):
    """Grouped restatement of moe_compute (where(topi == e) per expert) equals
    an independent token-by-token restatement, including ids that are absent
    from the expert dict (contribute nothing) and a skewed routing."""
    rng = np.random.default_rng(11 if skew else 12)
    T, k, n, H, Mi = 9, 3, 6, 64, 64
    experts = _rand_experts(rng, [0, 1, 2, 4, 5], H, Mi)        # expert 3 absent
    x = fmt.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    if skew:
        topi = np.stack([rng.permutation(n)[:k] for _ in range(T)])
        topi[:, 0] = 1                                            # every token hits expert 1
    else:
        topi = np.stack([rng.permutation(n)[:k] for _ in range(T)])
    scores = rng.random((T, k)).astype(np.float32)
    a = ops.moe_prefill_ref(x, topi, scores, experts)
    b = ops.moe_prefill_tokenwise_ref(x, topi, scores, experts)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-9)
    assert np.any(topi == 3)                                      # the absent id really occurs


def test_moe_prefill_ref_single_expert_weight_one_is_forward_chain():
    """One slot, one expert, score 1: the output is bf16 of the plain
    forward -> silu*mul -> forward chain of the reference operators."""
    rng = np.random.default_rng(5)
    T, H, Mi = 4, 64, 96
    experts = _rand_experts(rng, [0], H, Mi)
    x = fmt.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    topi = np.zeros((T, 1), np.int64)
    out = ops.moe_prefill_ref(x, topi, np.ones((T, 1), np.float32), experts)
    (gwp, gws), (uwp, uws), (dwp, dws) = experts[0]
    g = ops.forward_ref(x, gwp, gws).astype(np.float32)
    u = ops.forward_ref(x, uwp, uws).astype(np.float32)
    y = ops.forward_ref(ops.silu_mul_f32(g, u), dwp, dws)
    np.testing.assert_array_equal(out, fmt.bf16_round(fmt.bf16_round(y)).astype(np.float64))


# --------------------------------------------------------------------- GPU routing oracle
@pytest.mark.parametrize("n,k", [(128, 8), (60, 1), (256, 32), (1024, 8), (8, 8), (65, 3)])
def test_route_topk_np_matches_torch(n, k):
    """The numpy restatement against the reference's own calls (torch softmax,
    topk, renormalise on CPU): identical ids, weights to a few ulp."""
    rng = np.random.default_rng(n * 7 + k)
    lg = (rng.standard_normal((64, n)) * 3).astype(np.float32)
    ti, tv = ops.route_topk_np(lg, k)
    ri, rv = ops.route_ref(lg, k)
    assert np.array_equal(ti, ri)
    assert np.abs(tv - rv).max() <= 1e-6 * np.abs(rv).max()
    _, raw = ops.route_topk_np(lg, k, renorm=False)
    p = np.exp(lg - lg.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.allclose(raw, np.sort(p, -1)[:, ::-1][:, :k], rtol=1e-5, atol=0)


def test_route_topk_np_special_cases():
    # all-equal logits: ties go to the lower index, weights 1/k
    ti, tv = ops.route_topk_np(np.zeros((2, 16), np.float32), 4)
    assert np.array_equal(ti, [[0, 1, 2, 3]] * 2) and np.allclose(tv, 0.25)
    # -inf logits (masked experts) are never chosen while finite ones remain
    lg = np.full((1, 10), -np.inf, np.float32)
    lg[0, [7, 2, 9]] = [1.0, 3.0, 2.0]
    ti, tv = ops.route_topk_np(lg, 3)
    assert np.array_equal(ti, [[2, 9, 7]])
    e = np.exp(np.array([3.0, 2.0, 1.0]) - 3.0)
    assert np.allclose(tv[0], e / e.sum(), rtol=1e-6)
    # k == n: a full descending sort; renormalised weights are the softmax itself
    lg = np.array([[0.5, -1.0, 2.0, 0.0]], np.float32)
    ti, tv = ops.route_topk_np(lg, 4)
    assert np.array_equal(ti, [[2, 0, 3, 1]])
    p = np.exp(lg[0] - 2.0)
    assert np.allclose(tv[0], (p / p.sum())[[2, 0, 3, 1]], rtol=1e-6)
    # one dominant logit: weight ~1 on it
    lg = np.zeros((1, 32), np.float32)
    lg[0, 11] = 40.0
    ti, tv = ops.route_topk_np(lg, 8)
    assert ti[0, 0] == 11 and tv[0, 0] > 0.999999 and np.array_equal(ti[0, 1:], np.arange(7))
