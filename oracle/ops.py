"""Per-operator CPU references for the MXFP4 MoE hot path -- test infrastructure.

Each function restates what one reference operator computes, on dequantized
operands in float64, so that the HIP kernels (fp32 accumulation, different
summation order) can be compared under the stated tolerance.  Quantizer and
index outputs are compared bit-exactly.

Reference operators restated:
  prequant        src/ext/mxfp4_decode.cu:24-50, binding mxfp4_decode_binding.cpp:65-81
  forward         src/ext/mxfp4_linear.cu:106-198, binding mxfp4_binding.cpp:21-45
  lin_pq          src/ext/mxfp4_decode.cu:135-170, binding mxfp4_decode_binding.cpp:84-98
  moe_gateup      src/ext/mxfp4_decode.cu:177-212, binding mxfp4_decode_binding.cpp:101-120
  moe_down        src/ext/mxfp4_decode.cu:218-279, binding mxfp4_decode_binding.cpp:123-142
  moe_combine     src/ext/mxfp4_decode.cu:285-299, binding mxfp4_decode_binding.cpp:145-158
  routing         runtime/model_runner_v2.py:100-106,189-192,272-275
  moe_compute     runtime/model_runner_v2.py:108-122 (prefill / batched grouped MoE)
  token-major tables  runtime/model_runner_v2.py:197-206,279-286
  dequant+BF16 layer  runtime/model_runner.py:99-132 (the CPU baseline)
"""
import numpy as np

from . import mxfp4 as fmt


def prequant_ref(x):
    """bf16-valued (M, K) -> (xq (M, Kp/2) u8, xsc (M, Kp/32) u8), Kp = ceil32(K).
    Per 32-block of the bf16 row the fp4_format rule; the tail of the last
    block is zero.  For odd K the last element is packed (quant/fp4_format.py
    contract) rather than dropped as src/ext/mxfp4_decode.cu:46 does."""
    return fmt.quantize_rows(np.asarray(x, np.float32))


def forward_act_quant_ref(x, kp):
    """Activations of `forward`: rounded to fp16 first
    (src/ext/mxfp4_binding.cpp:31), then quantized per 32-block over the
    weight's Kp (src/ext/mxfp4_linear.cu:129-144, zero beyond K)."""
    return fmt.quantize_rows(fmt.f16_round(x), kp=kp)


def gemm_ref(a_deq, w_deq):
    """y = A @ W^T in float64 on dequantized operands."""
    return np.asarray(a_deq, np.float64) @ np.asarray(w_deq, np.float64).T


def lin_pq_ref(xq, xsc, wp, wsc):
    """y (M, N) = dequant(xq) @ dequant(W)^T over the full Kp (the reference
    kernel loops kk < Kp and relies on zero-padded activations)."""
    return gemm_ref(fmt.dequant_rows(xq, xsc), fmt.dequant_rows(wp, wsc))


def lin_pq_ref_chunked(xq, xsc, wp, wsc, rows=8192):
    """lin_pq_ref over row chunks of W (float64 dequant of one chunk at a
    time) for very tall weights such as a 151,936-row lm_head."""
    a = fmt.dequant_rows(xq, xsc).astype(np.float64)
    out = np.empty((a.shape[0], wp.shape[0]), np.float64)
    for r0 in range(0, wp.shape[0], rows):
        w = fmt.dequant_rows(wp[r0:r0 + rows], wsc[r0:r0 + rows]).astype(np.float64)
        out[:, r0:r0 + rows] = a @ w.T
    return out


def forward_ref(x, wp, wsc):
    kp = wp.shape[1] * 2
    xq, xsc = forward_act_quant_ref(x, kp)
    return lin_pq_ref(xq, xsc, wp, wsc)


def moe_gateup_ref(xq, xsc, wps, wscs, E, M, N):
    """gu (M*E, 2N): row m*E+e, columns [proj*N, proj*N+N) use the weight at
    token-major table index m*2E + proj*E + e (src/ext/mxfp4_decode.cu:187-195,211)."""
    a = fmt.dequant_rows(xq, xsc).astype(np.float64)
    gu = np.zeros((M * E, 2 * N), np.float64)
    for m in range(M):
        for proj in range(2):
            for e in range(E):
                t = m * 2 * E + proj * E + e
                w = fmt.dequant_rows(wps[t], wscs[t]).astype(np.float64)
                gu[m * E + e, proj * N:(proj + 1) * N] = w[:N] @ a[m, :w.shape[1]]
    return gu


def silu_mul_f32(g, u):
    """h = g / (1 + exp(-g)) * u in fp32 (src/ext/mxfp4_decode.cu:258)."""
    g = np.asarray(g, np.float32)
    u = np.asarray(u, np.float32)
    with np.errstate(over="ignore"):
        return ((g / (np.float32(1.0) + np.exp(-g))) * u).astype(np.float32)


def moe_down_h_ref(gu, E, M, K):
    """fp32 h rows (M*E, K) that moe_down quantizes."""
    gu = np.asarray(gu, np.float32)
    return silu_mul_f32(gu[:, :K], gu[:, K:2 * K])


def moe_down_ref(gu, wps, wscs, E, M, N, K, h=None):
    """yd (M*E, N): h = silu(gate)*up in fp32, quantized per 32-block to MXFP4
    (zero beyond K), then multiplied with the down weight of table index m*E+e
    (src/ext/mxfp4_decode.cu:218-279).  `h` may be supplied (e.g. the exact
    fp32 h the device computed) to separate SiLU ulps from the quantizer."""
    kp = wps[0].shape[1] * 2
    h = moe_down_h_ref(gu, E, M, K) if h is None else np.asarray(h, np.float32)
    hq, hs = fmt.quantize_rows(h, kp=kp)
    hd = fmt.dequant_rows(hq, hs).astype(np.float64)
    yd = np.zeros((M * E, N), np.float64)
    for z in range(M * E):
        w = fmt.dequant_rows(wps[z], wscs[z]).astype(np.float64)
        yd[z] = w[:N] @ hd[z]
    return yd


def moe_combine_ref(yd, w, M):
    """out[m, c] = sum_{e < min(E, 8)} w[m, e] * yd[m*E+e, c]; slots past 8 are
    ignored (src/ext/mxfp4_decode.cu:296).  Sequential fp32 order e = 0..7."""
    yd = np.asarray(yd, np.float32)
    w = np.asarray(w, np.float32).reshape(M, -1)
    E = w.shape[1]
    out = np.zeros((M, yd.shape[1]), np.float32)
    for m in range(M):
        acc = np.zeros(yd.shape[1], np.float32)
        for e in range(min(E, 8)):
            acc = (acc + w[m, e] * yd[m * E + e]).astype(np.float32)
        out[m] = acc
    return out


def route_ref(logits, k=8, renorm=True):
    """softmax(fp32) -> top-k (descending, torch.topk) -> renormalise.
    runtime/model_runner_v2.py:189-192 (decode) / :272-275 (batch).
    Uses the container's torch on CPU; returns (topi int64 (T,k), topv fp32)."""
    import torch
    lg = torch.as_tensor(np.asarray(logits, np.float32))
    probs = torch.softmax(lg, dim=-1)
    topv, topi = torch.topk(probs, k, dim=-1)
    if renorm:
        topv = topv / topv.sum(dim=-1, keepdim=True)
    return topi.numpy().astype(np.int64), topv.numpy().astype(np.float32)


def route_bruteforce(logits, k=8):
    """Index-only brute force: per row, experts ordered by probability
    descending, ties by lower index (the order torch.topk gives on CPU for
    distinct values).  Used to pin route_ref's indices."""
    lg = np.asarray(logits, np.float64)
    out = np.empty((lg.shape[0], k), np.int64)
    for t in range(lg.shape[0]):
        order = sorted(range(lg.shape[1]), key=lambda j: (-lg[t, j], j))
        out[t] = order[:k]
    return out


def token_major_tables(topi, n_tokens, k):
    """Token-major slot order the grouped ops consume
    (runtime/model_runner_v2.py:279-286): for token m the gate/up table holds
    [gate(ids[m*k+0..k-1]), up(same)] and the down table [down(same)].
    Returns (gateup_index (2kM,), down_index (kM,)) as (expert, proj) pairs
    encoded expert*2+proj for gate/up and expert for down."""
    ids = np.asarray(topi, np.int64).reshape(n_tokens, k)
    gu, dn = [], []
    for m in range(n_tokens):
        gu += [int(e) * 2 + 0 for e in ids[m]]
        gu += [int(e) * 2 + 1 for e in ids[m]]
        dn += [int(e) for e in ids[m]]
    return np.array(gu, np.int64), np.array(dn, np.int64)


def route_topk_np(logits, k=8, renorm=True):
    """numpy restatement of the routing of runtime/model_runner_v2.py:189-192
    (softmax in fp32 -> top-k -> renormalise): max, exp(l - max), sum,
    divide; top-k descending with exact ties broken towards the lower index
    (torch.topk leaves their order unspecified); the renormalisation sums the
    k winners in rank order.  Returns (topi int64 (M, k), topv fp32 (M, k))."""
    lg = np.atleast_2d(np.asarray(logits, np.float32))
    mx = lg.max(axis=-1, keepdims=True)
    e = np.exp((lg - mx).astype(np.float32)).astype(np.float32)
    s = e.sum(axis=-1, dtype=np.float32, keepdims=True)
    p = (e / s).astype(np.float32)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    topv = np.take_along_axis(p, order, axis=-1)
    if renorm:
        ts = np.zeros((p.shape[0], 1), np.float32)
        for r in range(k):
            ts = (ts + topv[:, r:r + 1]).astype(np.float32)
        topv = (topv / ts).astype(np.float32)
    return order.astype(np.int64), topv.astype(np.float32)


def group_by_expert(topi):
    """Token->expert grouping for the M<=16 grouped path.

    The (token, slot) pairs of topi (M, k) are sorted stably by expert id.
    Returns (experts (G,) ascending distinct ids, offsets (G+1,),
    pair_token (M*k,), pair_slot (M*k,)) where pairs offsets[g]:offsets[g+1]
    belong to experts[g] in ascending (token, slot) order.  This is the
    bookkeeping the reference builds implicitly with torch.where(topi == e)
    (runtime/model_runner_v2.py:111) and the token-major tables (:279-286)."""
    ids = np.asarray(topi, np.int64)
    M, k = ids.shape
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    experts, counts = np.unique(flat, return_counts=True)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    return experts, offsets, (order // k).astype(np.int64), (order % k).astype(np.int64)


def decode_layer_ref(x, topi, topv, experts):
    """Fused decode MoE layer on un-quantized activations, float64:
    out = sum_e w_e * Wd_e (silu(Wg_e x) * (Wu_e x)) with dequantized weights
    (runtime/model_runner.py:128-131 semantics computed in high precision).

    x (M, H) activations (bf16 values), topi/topv (M, k),
    experts: dict id -> ((gwp, gsc), (uwp, usc), (dwp, dsc)).
    Returns out (M, H) float64."""
    x = np.asarray(x, np.float64)
    if x.ndim == 1:
        x = x[None]
    topi = np.asarray(topi).reshape(x.shape[0], -1)
    topv = np.asarray(topv, np.float64).reshape(x.shape[0], -1)
    cache = {}
    rows = []
    for m in range(x.shape[0]):
        acc = None
        for s in range(topi.shape[1]):
            e = int(topi[m, s])
            if e not in cache:
                (gwp, gsc), (uwp, usc), (dwp, dsc) = experts[e]
                cache[e] = (fmt.dequant_rows(gwp, gsc).astype(np.float64),
                            fmt.dequant_rows(uwp, usc).astype(np.float64),
                            fmt.dequant_rows(dwp, dsc).astype(np.float64))
            wg, wu, wd = cache[e]
            H = wg.shape[1]
            g = wg @ x[m, :H]
            u = wu @ x[m, :H]
            h = g / (1.0 + np.exp(-g)) * u
            y = wd[:, :h.shape[0]] @ h
            acc = topv[m, s] * y if acc is None else acc + topv[m, s] * y
        rows.append(acc)
    return np.stack(rows)


def moe_prefill_ref(x, topi, scores, experts, bf16_steps=True, ambiguous=None):
    """ModelRunnerV2.moe_compute (runtime/model_runner_v2.py:108-122) on the
    operands the op consumes, float64 accumulation:
      for e in sorted(experts): idx, slots = where(topi == e)           (:111)
        g, u = forward(x[idx], gate_e / up_e)   x -> fp16 -> MXFP4      (:116-117)
        hh = silu(g) * u  (fp32)  -> forward(hh, down_e): fp16 -> MXFP4  (:118-119)
        y = bf16(y); out[idx] += bf16(y * bf16(score))                  (:119-120)
    experts: {e: ((gate_wp, gate_ws), (up_wp, up_ws), (down_wp, down_ws))}.
    Ids absent from `experts` contribute nothing.  With bf16_steps the two
    bf16 roundings of y and y*score are applied; the sum over slots is kept in
    float64 (the reference's bf16 index_add_ order is not restated: parity of
    that last rounding is by tolerance).  Returns float64 (T, H).

    If `ambiguous` is a boolean array of shape (T,), tokens are flagged in it
    whose MXFP4 h quantization is not robust: h * (1 +- 1e-5) quantizes to
    other codes or scales than h.  Any fp32 implementation (the reference's
    included) may legitimately round such an h the other way."""
    x = np.asarray(x, np.float32)
    topi = np.asarray(topi, np.int64)
    scores = fmt.bf16_round(np.asarray(scores, np.float32))
    T, H = x.shape
    out = np.zeros((T, H), np.float64)
    xq, xs = forward_act_quant_ref(x, H)
    xd = fmt.dequant_rows(xq, xs).astype(np.float64)
    for e in sorted(experts):
        idx, slots = np.nonzero(topi == e)
        if idx.size == 0:
            continue
        (gwp, gws), (uwp, uws), (dwp, dws) = experts[e]
        g = (xd[idx] @ fmt.dequant_rows(gwp, gws).astype(np.float64).T).astype(np.float32)
        u = (xd[idx] @ fmt.dequant_rows(uwp, uws).astype(np.float64).T).astype(np.float32)
        hh = silu_mul_f32(g, u)
        hq, hs = forward_act_quant_ref(hh, dwp.shape[1] * 2)
        if ambiguous is not None:
            for f in (1.0 + 1e-5, 1.0 - 1e-5):
                q2, s2 = forward_act_quant_ref(hh * np.float32(f), dwp.shape[1] * 2)
                bad = np.any(q2 != hq, axis=1) | np.any(s2 != hs, axis=1)
                ambiguous[idx[bad]] = True
        y = fmt.dequant_rows(hq, hs).astype(np.float64) @ fmt.dequant_rows(dwp, dws).astype(np.float64).T
        s = scores[idx, slots].astype(np.float64)[:, None]
        if bf16_steps:
            contrib = fmt.bf16_round((fmt.bf16_round(y).astype(np.float64) * s).astype(np.float32))
        else:
            contrib = y * s
        np.add.at(out, idx, contrib.astype(np.float64))
    return out


def moe_prefill_tokenwise_ref(x, topi, scores, experts):
    """The same operator restated token by token (no grouping): for each
    token t and slot k, y = forward(h(x_t)) with expert topi[t, k], summed
    over k.  An independent loop structure to pin moe_prefill_ref's
    idx/slot bookkeeping."""
    x = np.asarray(x, np.float32)
    topi = np.asarray(topi, np.int64)
    scores = fmt.bf16_round(np.asarray(scores, np.float32))
    T, H = x.shape
    out = np.zeros((T, H), np.float64)
    for t in range(T):
        for k in range(topi.shape[1]):
            e = int(topi[t, k])
            if e not in experts:
                continue
            (gwp, gws), (uwp, uws), (dwp, dws) = experts[e]
            g = forward_ref(x[t:t + 1], gwp, gws).astype(np.float32)
            u = forward_ref(x[t:t + 1], uwp, uws).astype(np.float32)
            y = forward_ref(silu_mul_f32(g, u), dwp, dws)[0]
            out[t] += fmt.bf16_round((fmt.bf16_round(y).astype(np.float64) * scores[t, k]).astype(np.float32))
    return out


def dequant_bf16_moe_layer_torch(x, topi, topv, experts_deq_bf16=None, experts=None):
    """The reference's dequant + BF16 expert path on the CPU with torch
    (runtime/model_runner.py:128-131; dequant runtime/weight_store.py:27-44).

    Either pre-dequantized bf16 weights {e: (Wg, Wu, Wd)} or packed experts
    {e: ((gwp, gsc), (uwp, usc), (dwp, dsc))} (dequantized here, timed).
    x: torch bf16 (M, H).  Returns torch bf16 (M, H)."""
    import torch
    import torch.nn.functional as F
    topi = torch.as_tensor(np.asarray(topi)).reshape(x.shape[0], -1)
    topv = torch.as_tensor(np.asarray(topv, np.float32)).reshape(x.shape[0], -1)
    out = torch.zeros_like(x)
    for e in torch.unique(topi).tolist():
        if experts_deq_bf16 is not None:
            wg, wu, wd = experts_deq_bf16[e]
        else:
            wg, wu, wd = (dequant_bf16_torch(*experts[e][j]) for j in range(3))
        idx, slots = torch.where(topi == e)
        xt = x[idx]
        hh = F.silu(F.linear(xt, wg)) * F.linear(xt, wu)
        y = F.linear(hh, wd)
        out.index_add_(0, idx, (y * topv[idx, slots].unsqueeze(-1)).to(x.dtype))
    return out


_TABLE = None


def dequant_bf16_torch(wp, wsc, k=None):
    """Torch-CPU dequant (runtime/weight_store.py:27-44) -> bf16 (n, k)."""
    import torch
    global _TABLE
    if _TABLE is None:
        _TABLE = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    wp = torch.as_tensor(np.asarray(wp))
    wsc = torch.as_tensor(np.asarray(wsc))
    n, half = wp.shape
    kp = half * 2
    codes = torch.empty(n, kp, dtype=torch.uint8)
    codes[:, 0::2] = wp & 0xF
    codes[:, 1::2] = wp >> 4
    codes = codes.view(n, kp // 32, 32)
    sign = torch.where((codes & 0x8) != 0, -1.0, 1.0)
    vals = _TABLE[(codes & 0x7).long()]
    scales = torch.exp2(wsc.float() - 127.0)
    rec = (sign * vals * scales[..., None]).reshape(n, kp)
    if k is not None:
        rec = rec[:, :k]
    return rec.to(torch.bfloat16)


def cos_sim(a, b):
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    return float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def max_rel(y, ref):
    """Norm-wise max relative error: max|y - ref| / max|ref|."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max()
    return float(np.abs(y - ref).max() / den) if den > 0 else float(np.abs(y).max())
