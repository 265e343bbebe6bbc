"""CPU restatement of the reference's decode step -- test infrastructure
(only tests/ use it).

Reference:
  rms_norm          runtime/model_runner.py:20-25
  apply_rope        runtime/model_runner.py:28-41 (half layout, theta)
  dequant_rows_gpu  runtime/weight_store.py:47-65 (embedding rows)
  forward_decode    runtime/model_runner_v2.py:130-217 (one token)
  forward_batch     runtime/model_runner_v2.py:220-300 (M tokens of one sequence)
  greedy next token runtime/decode_v2.py:71 (logits[-1].argmax())

numpy float32 where the reference computes in fp32 and bf16 rounding where it
rounds; the matmuls (lin_pq, attention, MoE) are the float64 oracles of
oracle/ops.py and oracle/attn.py.  Differences to the GPU step come from
fp32 accumulation order and the transcendental functions (rsqrt, cos, sin,
exp), so the comparison is to a tolerance.
"""
import numpy as np

from . import attn as attn_ref
from . import mxfp4 as fmt
from . import ops

bf16 = fmt.bf16_round


def rms_norm_ref(x, w, eps, bf16_input=True):
    """runtime/model_runner.py:20-25: xf = x.float(); xf * rsqrt(mean(xf^2) + eps);
    cast back to the input dtype; times the bf16 weight (bf16 * bf16 -> bf16
    for bf16 input, fp32 for fp32 input -- the caller's .bfloat16() then
    rounds).  Returns bf16 values as float32."""
    xf = np.asarray(x, np.float32)
    var = np.mean(xf.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    y = (xf * r).astype(np.float32)
    if bf16_input:
        y = bf16(y)
    return bf16((y * np.asarray(w, np.float32)).astype(np.float32))


def rope_ref(x, positions, theta):
    """runtime/model_runner.py:28-41 on x (T, nh, D) bf16 values: fp32
    inv_freq and angles, x * cos + rotate_half(x) * sin in fp32, to bf16."""
    x = np.asarray(x, np.float32)
    D = x.shape[-1]
    inv = (np.float32(1.0) / np.power(np.float32(theta), np.arange(0, D, 2, dtype=np.float32) / np.float32(D))).astype(np.float32)
    freqs = (np.asarray(positions, np.float32)[:, None] * inv[None, :]).astype(np.float32)
    cos = np.cos(freqs.astype(np.float64)).astype(np.float32)
    sin = np.sin(freqs.astype(np.float64)).astype(np.float32)
    cos = np.concatenate([cos, cos], axis=-1)[:, None, :]
    sin = np.concatenate([sin, sin], axis=-1)[:, None, :]
    rot = np.concatenate([-x[..., D // 2:], x[..., : D // 2]], axis=-1)
    return bf16(((x * cos).astype(np.float32) + (rot * sin).astype(np.float32)).astype(np.float32))


def embed_ref(wp, ws, ids, K):
    """runtime/weight_store.py:47-65: rows ids of an MXFP4 matrix, dequantized, to bf16."""
    ids = np.asarray(ids)
    return bf16(fmt.dequant_rows(wp[ids], ws[ids], K).astype(np.float32))


def argmax_ref(logits):
    """First index of each row's maximum (torch.argmax)."""
    return np.argmax(np.asarray(logits), axis=-1).astype(np.int32)


def layer_ref(lw, cfg, x, base, kvk_l, kvv_l, fused_moe, kv_codec=0, teacher=None, trace=None):
    """One decoder layer of the step (runtime/model_runner_v2.py:147-208 for
    M = 1, :238-297 for M > 1) on the residual stream x (M, H) bf16 values of
    tokens at positions base..base+M-1.  lw: that layer's weights (as in
    step_ref), kvk_l / kvv_l: its (max_pos, Hkv, D) caches, updated in place.
    Returns the residual stream after the layer (bf16 values).

    teacher: optional dict of another implementation's intermediates of this
    layer; each given one replaces this function's own value from that point
    on, so every stage can be compared on identical inputs: "qkv" (M, (Hq +
    2 Hkv) D) fp32 projection, "x_mid" the residual after the attention block,
    "hp2" the post-attention RMSNorm output (bf16 values), "glog" the router
    logits.  trace: optional dict that receives this function's own
    intermediates under the same names plus "oproj", "topi", "topv", "moe"."""
    teacher = teacher or {}
    tr = trace if trace is not None else {}
    x = np.asarray(x, np.float32)
    M = x.shape[0]
    D, Hq, Hkv, E, H = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads, cfg.top_k, cfg.hidden
    eps = cfg.rms_eps
    pos = np.arange(base, base + M)
    hp = rms_norm_ref(x, lw["in_norm"], eps)
    hq, hs = fmt.quantize_rows(hp)
    qkv = ops.lin_pq_ref(hq, hs, *lw["qkv"]).astype(np.float32)
    tr["qkv"] = qkv
    if "qkv" in teacher:
        qkv = np.asarray(teacher["qkv"], np.float32).reshape(M, -1)
    q = qkv[:, : Hq * D].reshape(M, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(M, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].reshape(M, Hkv, D)
    qn = rms_norm_ref(q, lw["q_norm"], eps, bf16_input=False)
    kn = rms_norm_ref(k, lw["k_norm"], eps, bf16_input=False)
    qr, kr = rope_ref(qn, pos, cfg.rope_theta), rope_ref(kn, pos, cfg.rope_theta)
    attn_ref.kv_write_ref(kr, bf16(v), kvk_l, kvv_l, base, kv_codec)
    o_att, _ = attn_ref.attn_decode_ref(qr, kvk_l, kvv_l, base)
    of = bf16(o_att.astype(np.float32)).reshape(M, Hq * D)
    aq, as_ = fmt.quantize_rows(of)
    o = ops.lin_pq_ref(aq, as_, *lw["o"]).astype(np.float32)
    tr["oproj"] = o
    x = bf16((x + bf16(o)).astype(np.float32))
    tr["x_mid"] = x
    if "x_mid" in teacher:
        x = np.asarray(teacher["x_mid"], np.float32).reshape(M, H)
    hp2 = rms_norm_ref(x, lw["post_norm"], eps)
    tr["hp2"] = hp2
    if "hp2" in teacher:
        hp2 = np.asarray(teacher["hp2"], np.float32).reshape(M, H)
    h2q, h2s = fmt.quantize_rows(hp2)
    glog = ops.lin_pq_ref(h2q, h2s, *lw["gate"]).astype(np.float32)
    tr["glog"] = glog
    if "glog" in teacher:
        glog = np.asarray(teacher["glog"], np.float32).reshape(M, -1)
    topi, topv = ops.route_topk_np(glog, E, renorm=True)
    tr["topi"], tr["topv"] = topi, topv
    if fused_moe:
        moe = ops.decode_layer_ref(hp2, topi, topv, lw["experts"]).astype(np.float32)
    else:
        ex = lw["experts"]
        # token-major table: entry m*2E + proj*E + e (runtime/model_runner_v2.py:279-286)
        tw = [ex[int(e)][proj][0] for m in range(M) for proj in (0, 1) for e in topi[m]]
        ts = [ex[int(e)][proj][1] for m in range(M) for proj in (0, 1) for e in topi[m]]
        gu = ops.moe_gateup_ref(h2q, h2s, tw, ts, E, M, cfg.moe_inter)
        yd = ops.moe_down_ref(gu, [ex[int(e)][2][0] for e in topi.reshape(-1)],
                              [ex[int(e)][2][1] for e in topi.reshape(-1)], E, M, H, cfg.moe_inter)
        moe = ops.moe_combine_ref(yd, topv.astype(np.float32), M).astype(np.float32)
    tr["moe"] = moe
    return bf16((x + bf16(moe)).astype(np.float32))


def head_ref(w, cfg, x):
    """Final RMSNorm -> MXFP4 -> lm_head (runtime/model_runner_v2.py:210-217,
    :296-300): logits (M, V) float64, computed over row chunks of the lm_head
    so a vocabulary of 151,936 rows stays within a few hundred MB."""
    xf = rms_norm_ref(x, w["final_norm"], cfg.rms_eps)
    fq, fs = fmt.quantize_rows(xf)
    return ops.lin_pq_ref_chunked(fq, fs, *w["lm_head"])


def step_ref(w, cfg, ids, base, kvk, kvv, fused_moe, x_teacher=None, kv_codec=0):
    """One step of M = len(ids) tokens at positions base..base+M-1.

    w: dict of numpy arrays (keys as DecodeStep's weights: embed, layers[l]
    {in_norm, qkv, q_norm, k_norm, o, post_norm, gate, experts}, final_norm,
    lm_head; Packed weights as (wp, ws) pairs, experts as {e: ((gwp, gws),
    (uwp, uws), (dwp, dws))}).  kvk, kvv: (L, max_pos, Hkv, D) uint8 caches,
    updated in place.  fused_moe: the MoE on bf16 activations
    (decode_layer_ref, the one-token fused path) or, False, the drop-in ops on
    MXFP4 activations (forward_batch).  x_teacher: optional list of the
    residual stream after each layer as another implementation computed it;
    layer l > 0 and the head then start from x_teacher[l-1] / x_teacher[-1]
    instead of this function's own value (teacher forcing, so each layer is
    compared on identical inputs).  kv_codec: the cache encoder, 0 the decode
    extension's kv_write (the graph runner, runtime/model_runner_v3.py:
    98-101), 1 torch's float8_e4m3fn (forward_batch,
    runtime/model_runner_v2.py:256-257).  Returns (logits (M, V) float64,
    [x after each layer] bf16 values)."""
    ids = np.asarray(ids)
    x = embed_ref(*w["embed"], ids, cfg.hidden)
    xs = []
    for l, lw in enumerate(w["layers"]):
        if x_teacher is not None and l > 0:
            x = np.asarray(x_teacher[l - 1], np.float32)
        x = layer_ref(lw, cfg, x, base, kvk[l], kvv[l], fused_moe, kv_codec)
        xs.append(x)
    if x_teacher is not None:
        x = np.asarray(x_teacher[-1], np.float32)
    return head_ref(w, cfg, x), xs


def step_ref_layers(w, cfg, ids, base, kvk, kvv, fused_moe, x_teacher, layers, kv_codec=0, stage_teacher=None):
    """Teacher-forced check of selected layers of one step: layer l starts
    from x_teacher[l-1] (layer 0 from the embedding of ids), and the head
    from x_teacher[-1].  w["layers"], kvk and kvv need hold only the
    selected layers (mappings l -> weights / (max_pos, Hkv, D) caches).
    stage_teacher: optional {l: teacher dict of layer_ref}.
    Returns (logits (M, V) float64, {l: x after layer l}, {l: trace})."""
    out, traces = {}, {}
    for l in layers:
        x = embed_ref(*w["embed"], np.asarray(ids), cfg.hidden) if l == 0 else x_teacher[l - 1]
        traces[l] = {}
        out[l] = layer_ref(w["layers"][l], cfg, x, base, kvk[l], kvv[l], fused_moe, kv_codec,
                           teacher=(stage_teacher or {}).get(l), trace=traces[l])
    return head_ref(w, cfg, np.asarray(x_teacher[-1], np.float32)), out, traces
