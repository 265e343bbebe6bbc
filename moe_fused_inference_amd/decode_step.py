"""A whole Qwen3-MoE-shaped decode step on this library's kernels.

The reference's step (runtime/model_runner_v2.py:130-217 forward_decode for
one token, :220-300 forward_batch for M tokens of one sequence, driven by the
greedy loop of runtime/decode_v2.py:64-71):

    x = embed_rows(ids)                                    (MXFP4 row dequant)
    per layer:
        hp  = rms_norm(x) -> MXFP4;  q, k, v = lin_pq(hp)   (one fused q|k|v weight)
        q, k = rms_norm per head (q_norm, k_norm), RoPE;  k, v -> FP8 KV cache
        o   = attn_decode(q, cache) -> bf16 -> MXFP4 -> lin_pq(o_proj)
        x   = x + bf16(o);  hp2 = rms_norm(x) -> MXFP4;  logits = lin_pq(gate)
        moe = softmax / top-k / renorm routing + experts + weighted combine
        x   = x + bf16(moe)
    logits = lin_pq(rms_norm(x));  next ids = argmax;  position += M

Every op is a kernel of this library; positions and token ids live in device
memory, so one step can be captured in a HIP graph and replayed step after
step (DecodeStep.capture).  MoE: M = 1 uses the fused one-launch layer with
in-kernel routing on the bf16 activations (mxfp4_moe_decode_layer_routed);
M > 1 uses route_topk + mxfp4_moe_decode_batch on MXFP4 activations, the
arithmetic of forward_batch's moe_gateup -> moe_down -> moe_combine chain in
two launches that read each routed expert once.  The KV cache holds E4M3 bytes with no extra scale, read
by attn_decode's codec; they are written the way the matching reference
step writes them: M = 1 with the decode extension's kv_write codec (the
graph runner, runtime/model_runner_v3.py:98-101), M > 1 with torch's
float8_e4m3fn conversion (forward_batch, runtime/model_runner_v2.py:256-257).
"""
import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from .moe_layer import (FusedRouterLayerCall, PostAttnLayerCall, RoutedLayerCall, StackedExperts, layer_status,
                        workspace as layer_workspace)


@dataclass
class ModelConfig:
    n_layers: int = 48
    hidden: int = 2048
    n_heads: int = 32
    n_kv_heads: int = 4
    head_dim: int = 128
    n_experts: int = 128
    top_k: int = 8
    moe_inter: int = 768
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def qkv_rows(self):
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


@dataclass
class Packed:
    """An MXFP4 weight (N, K): packed nibbles (N, Kp/2) and E8M0 codes (N, Kp/32)."""
    wp: torch.Tensor
    ws: torch.Tensor

    @property
    def n(self):
        return int(self.wp.shape[0])

    @property
    def k(self):
        return int(self.wp.shape[1]) * 2


@dataclass
class LayerWeights:
    in_norm: torch.Tensor          # bf16 (H,)
    qkv: Packed                    # ((Hq + 2 Hkv) D, H): q_proj | k_proj | v_proj rows
    q_norm: torch.Tensor           # bf16 (D,)
    k_norm: torch.Tensor           # bf16 (D,)
    o: Packed                      # (H, Hq D)
    post_norm: torch.Tensor        # bf16 (H,)
    gate: Packed                   # (n_experts, H) router
    experts: StackedExperts


@dataclass
class ModelWeights:
    embed: Packed                  # (V, H)
    layers: list
    final_norm: torch.Tensor       # bf16 (H,)
    lm_head: Packed                # (V, H)


def _quantize(w_bf16):
    """bf16 (N, K) -> Packed, with the library's bit-exact quantizer."""
    lib = _lib.load()
    n, k = w_bf16.shape
    kp = (k + 31) // 32 * 32
    wp = torch.empty((n, kp // 2), dtype=torch.uint8, device=w_bf16.device)
    ws = torch.empty((n, kp // 32), dtype=torch.uint8, device=w_bf16.device)
    _lib.check(lib.mxfp4_prequant(w_bf16.data_ptr(), k, n, k, kp, wp.data_ptr(), ws.data_ptr(),
                                  torch.cuda.current_stream().cuda_stream), "prequant")
    return Packed(wp, ws)


def synthetic_model(cfg, seed=0, device="cuda", std=0.02, experts=None):
    """Random-init weights of the given shape (no checkpoint): projections,
    router, experts, embedding and lm_head bf16 N(0, std) quantized to MXFP4;
    norm weights bf16 1 + N(0, std).  experts: optional list of per-layer
    StackedExperts to use instead of new random ones."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def rnd(n, k):
        return _quantize((torch.randn((n, k), generator=g, device=device) * std).bfloat16())

    def norm(n):
        return (1.0 + std * torch.randn(n, generator=g, device=device)).bfloat16()

    H, D, Mi, n_exp = cfg.hidden, cfg.head_dim, cfg.moe_inter, cfg.n_experts
    layers = []
    for li in range(cfg.n_layers):
        if experts is not None:
            layers.append(LayerWeights(in_norm=norm(H), qkv=rnd(cfg.qkv_rows, H), q_norm=norm(D), k_norm=norm(D),
                                       o=rnd(H, cfg.n_heads * D), post_norm=norm(H), gate=rnd(n_exp, H),
                                       experts=experts[li]))
            continue
        ex = {}
        for nm, (n, k) in (("gate", (Mi, H)), ("up", (Mi, H)), ("down", (H, Mi))):
            wp = torch.empty((n_exp, n, k // 2), dtype=torch.uint8, device=device)
            ws = torch.empty((n_exp, n, k // 32), dtype=torch.uint8, device=device)
            chunk = max(1, min(n_exp, (64 << 20) // (n * k * 4)))
            for e0 in range(0, n_exp, chunk):
                ce = min(chunk, n_exp - e0)
                p = rnd(ce * n, k)
                wp[e0:e0 + ce] = p.wp.view(ce, n, k // 2)
                ws[e0:e0 + ce] = p.ws.view(ce, n, k // 32)
            ex[nm + "_wp"], ex[nm + "_ws"] = wp, ws
        layers.append(LayerWeights(in_norm=norm(H), qkv=rnd(cfg.qkv_rows, H), q_norm=norm(D), k_norm=norm(D),
                                   o=rnd(H, cfg.n_heads * D), post_norm=norm(H), gate=rnd(n_exp, H),
                                   experts=StackedExperts(**ex)))
    return ModelWeights(embed=rnd(cfg.vocab, H), layers=layers, final_norm=norm(H), lm_head=rnd(cfg.vocab, H))


@dataclass
class _Bufs:
    tensors: dict = field(default_factory=dict)

    def __getattr__(self, k):
        try:
            return self.tensors[k]
        except KeyError:
            raise AttributeError(k)


class DecodeStep:
    """M tokens of one sequence per step (M = 1: forward_decode; M > 1:
    forward_batch).  ids (M,) int32 and the base position dpos (1,) int32
    stay on the device: each step reads them and leaves the greedy next
    tokens and dpos + M for the next step."""

    def __init__(self, model, cfg, M=1, max_pos=4096, device="cuda", fused_router=True, qkv_tail=True,
                 attn_front=True, attn_next=True):
        self.lib = _lib.load()
        self.model, self.cfg, self.M, self.max_pos = model, cfg, int(M), int(max_pos)
        self.kv_codec = 0 if self.M == 1 else 1   # kv_write's codec / torch float8_e4m3fn
        self.fused_norm = cfg.hidden == 2048 and self.M == 1   # at M > 1 the per-workgroup norm costs more than the launch it saves
        # M = 1: post-attention residual + RMSNorm + router inside the MoE launch
        # (mxfp4_moe_decode_layer_fused_router), one launch per layer fewer
        self.fused_router = (bool(fused_router) and self.M == 1 and cfg.hidden == 2048 and cfg.n_experts % 16 == 0
                             and cfg.n_experts <= 256)
        # with the fused router, the next layer's input residual + RMSNorm +
        # q|k|v projection also run in the MoE launch
        # (mxfp4_moe_decode_layer_fused_router_qkv): another launch per layer fewer
        self.qkv_tail = self.fused_router and bool(qkv_tail)
        # with the q|k|v tail, the attention merge and o_proj also run in the
        # MoE launch (mxfp4_decode_layer_post_attn; 32 heads of 128): two
        # launches per layer in all
        self.attn_front = self.qkv_tail and bool(attn_front) and cfg.n_heads == 32 and cfg.head_dim == 128
        # and with the front, the next layer's attention chunk pass too: one
        # launch per layer (8 query heads per kv head, max_pos * kv heads <= 32768)
        self.attn_next = (self.attn_front and bool(attn_next) and cfg.n_heads == 8 * cfg.n_kv_heads
                          and ((max_pos + 63) // 64) * cfg.n_kv_heads <= 512)
        self._fr_calls = {}
        c = cfg
        if c.head_dim != 128:
            raise RuntimeError("head_dim must be 128 (attention kernels)")
        if c.hidden % 2048:
            raise RuntimeError("hidden must be a multiple of 2048 (norm kernel)")
        M, H, D, Hq, Hkv = self.M, c.hidden, c.head_dim, c.n_heads, c.n_kv_heads
        f32, bf16, u8, i32 = torch.float32, torch.bfloat16, torch.uint8, torch.int32
        t = {}

        def buf(name, shape, dt):
            t[name] = torch.zeros(shape, dtype=dt, device=device)

        buf("ids", (M,), i32)
        buf("dpos", (1,), i32)
        buf("x", (M, H), bf16)
        buf("x2", (M, H), bf16)
        buf("x3", (M, H), bf16)
        buf("y", (M, H), bf16)
        buf("yq", (M, H // 2), u8)
        buf("ys", (M, H // 32), u8)
        buf("qkv", (M, c.qkv_rows), f32)
        buf("qkv2", (M, c.qkv_rows), f32)   # odd layers' q|k|v with the q|k|v tail
        buf("aq", (M, Hq * D // 2), u8)
        buf("as_", (M, Hq * D // 32), u8)
        buf("oproj", (M, H), f32)
        buf("glog", (M, c.n_experts), f32)
        buf("moe", (M, H), f32)
        buf("logits", (M, c.vocab), f32)
        nb = self.lib.mxfp4_argmax_workspace_size(M, c.vocab)
        buf("arg_ws", ((nb + 255) // 256 * 256,), u8)   # zero-filled once; each call leaves it so
        nb = self.lib.mxfp4_attn_decode_workspace_size(M, Hq, self.max_pos)
        buf("attn_ws", ((nb + 15) // 16 * 16,), u8)
        buf("attn_ws2", ((nb + 15) // 16 * 16,) if M == 1 else (16,), u8)   # odd layers' chunk records (attn_next)
        # KV cache of every layer: (L, max_pos, Hkv, D) E4M3 bytes
        buf("kvk", (c.n_layers, self.max_pos, Hkv, D), u8)
        buf("kvv", (c.n_layers, self.max_pos, Hkv, D), u8)
        if M == 1:
            self.layer_ws = layer_workspace(c.top_k, c.moe_inter, H, device)
            self.moe_calls = [RoutedLayerCall(t["y"][0], t["glog"][0], c.top_k, lw.experts, t["moe"][0], None,
                                              self.layer_ws) for lw in model.layers]
        else:
            E = c.top_k
            buf("rid", (M, E), i32)
            buf("rw", (M, E), f32)
            nb = self.lib.mxfp4_moe_decode_batch_workspace_size(M, E, c.moe_inter)
            buf("moe_ws", ((nb + 15) // 16 * 16,), u8)
        self.b = _Bufs(t)

    # ------------------------------------------------------------------ state
    def set_state(self, ids, pos):
        """Token ids (M,) and the base position of the next step."""
        self.b.ids.copy_(torch.as_tensor(ids, dtype=torch.int32).reshape(-1))
        self.b.dpos.fill_(int(pos))

    def fill_cache(self, upto, seed=1):
        """Synthetic context: random E4M3 bytes for positions [0, upto) of
        every layer's cache (codes of |v| < 2, no NaN code)."""
        g = torch.Generator(device=self.b.kvk.device)
        g.manual_seed(seed)
        for kv in (self.b.kvk, self.b.kvv):
            r = torch.randint(0, 256, kv[:, :upto].shape, generator=g, device=kv.device, dtype=torch.int32)
            kv[:, :upto] = ((r & 0x80) | (r & 0x3F)).to(torch.uint8)   # exponent field <= 7: |v| < 2

    # ------------------------------------------------------------------ one step
    def _ck(self, rc, what):
        _lib.check(rc, what)

    def _lin(self, xq, xs, w, N, K, out, s):
        kp = (K + 31) // 32 * 32
        self._ck(self.lib.mxfp4_lin_pq(xq.data_ptr(), xs.data_ptr(), w.wp.data_ptr(), w.ws.data_ptr(), out.data_ptr(),
                                       self.M, N, K, kp, s), "lin_pq")

    def _norm_lin(self, x, resid, nw, x_out, keep, w, out, s):
        """rms_norm(x [+ resid]) -> MXFP4 -> lin_pq(w) in one launch at M = 1
        (H = 2048), else rmsnorm_quant + lin_pq.  keep:
        also leave y and its MXFP4 rows in the step buffers."""
        lib, c, b, M, H = self.lib, self.cfg, self.b, self.M, self.cfg.hidden
        ptr = (lambda t: t.data_ptr() if t is not None else None)
        if self.fused_norm:
            self._ck(lib.mxfp4_rmsnorm_lin_pq(x.data_ptr(), ptr(resid), nw.data_ptr(), c.rms_eps, M, H, ptr(x_out),
                                              ptr(b.y) if keep else None, ptr(b.yq) if keep else None,
                                              ptr(b.ys) if keep else None, w.wp.data_ptr(), w.ws.data_ptr(), w.n,
                                              out.data_ptr(), s), "rmsnorm_lin_pq")
        else:
            self._ck(lib.mxfp4_rmsnorm_quant(x.data_ptr(), ptr(resid), nw.data_ptr(), c.rms_eps, M, H, ptr(x_out),
                                             b.y.data_ptr(), b.yq.data_ptr(), b.ys.data_ptr(), s), "rmsnorm_quant")
            self._lin(b.yq, b.ys, w, w.n, H, out, s)

    def qkv_buf(self, l):
        """The buffer that holds layer l's q|k|v projection (M, qkv_rows) from
        before its attention to the end of the step (read it from an
        on_layer hook): with the q|k|v tail, layer l's projection is written
        by layer l-1's MoE launch, so odd and even layers alternate buffers."""
        return self.b.qkv2 if (self.qkv_tail and l % 2) else self.b.qkv

    def attn_ws_of(self, l):
        """The attention workspace holding layer l's chunk records: with the
        next layer's attention in each layer launch, odd and even layers
        alternate buffers (a launch merges one layer's records while it
        writes the next layer's)."""
        return self.b.attn_ws2 if (self.attn_next and l % 2) else self.b.attn_ws

    def _attn_oproj(self, l, lw, qkv, s):
        """q/k head norm + RoPE, the step's KV rows and attention in one pass,
        its output straight to MXFP4 of bf16(o) (the raw scores are not kept),
        then o_proj into b.oproj."""
        lib, c, b, M = self.lib, self.cfg, self.b, self.M
        H, D, Hq, Hkv = c.hidden, c.head_dim, c.n_heads, c.n_kv_heads
        kvk, kvv = b.kvk[l], b.kvv[l]
        self._ck(lib.mxfp4_attn_decode_fused(qkv.data_ptr(), lw.q_norm.data_ptr(), lw.k_norm.data_ptr(),
                                             c.rms_eps, c.rope_theta, kvk.data_ptr(), kvv.data_ptr(),
                                             b.dpos.data_ptr(), None, None, b.aq.data_ptr(),
                                             b.as_.data_ptr(), M, Hq, Hkv, D, self.max_pos, self.kv_codec,
                                             b.attn_ws.data_ptr(), b.attn_ws.numel(), s), "attn_decode_fused")
        self._lin(b.aq, b.as_, lw.o, H, Hq * D, b.oproj, s)

    def _layers_qkv_tail(self, on_layer, s):
        """The layers at M = 1 with the q|k|v tail: per layer the attention,
        o_proj and one MoE launch that also runs the router and the next
        layer's input norm + q|k|v; with attn_front, the attention's chunk
        pass and one launch for the rest (merge, o_proj, router, MoE, next
        q|k|v).  The residual stream rotates through three buffers (a
        launch's x, x_out and x_next are distinct).  Returns (x_out of the
        last layer, a free buffer)."""
        c, b, m = self.cfg, self.b, self.model
        xs = (b.x, b.x2, b.x3)
        L = len(m.layers)
        self._norm_lin(b.x, None, m.layers[0].in_norm, None, False, m.layers[0].qkv, self.qkv_buf(0), s)
        cur = 0                      # xs[cur]: the layer's input residual stream
        for l, lw in enumerate(m.layers):
            if self.attn_front and (l == 0 or not self.attn_next):
                aws = self.attn_ws_of(l)
                self._ck(self.lib.mxfp4_attn_decode_fused_partials(
                    self.qkv_buf(l).data_ptr(), lw.q_norm.data_ptr(), lw.k_norm.data_ptr(), c.rms_eps, c.rope_theta,
                    b.kvk[l].data_ptr(), b.kvv[l].data_ptr(), b.dpos.data_ptr(), 1, c.n_heads, c.n_kv_heads,
                    c.head_dim, self.max_pos, self.kv_codec, aws.data_ptr(), aws.numel(), s),
                    "attn_decode_fused_partials")
            elif not self.attn_front:
                self._attn_oproj(l, lw, self.qkv_buf(l), s)
            xo, xn = (cur + 1) % 3, (cur + 2) % 3
            call = self._fr_calls.get(("tail", l))
            if call is None:
                nxt = None
                if l + 1 < L:
                    nl = m.layers[l + 1]
                    nxt = (nl.in_norm, nl.qkv.wp, nl.qkv.ws, self.qkv_buf(l + 1)[0], xs[xn][0])
                if self.attn_front:
                    nat = None
                    if self.attn_next and l + 1 < L:
                        nl = m.layers[l + 1]
                        nat = (self.attn_ws_of(l + 1), b.kvk[l + 1], b.kvv[l + 1], nl.q_norm, nl.k_norm, c.n_kv_heads,
                               c.rope_theta, self.kv_codec)
                    call = PostAttnLayerCall(self.attn_ws_of(l), b.dpos, self.max_pos, lw.o.wp, lw.o.ws, b.oproj[0],
                                             xs[cur][0], lw.post_norm, c.rms_eps, lw.gate.wp, lw.gate.ws, c.top_k,
                                             lw.experts, b.moe[0], self.layer_ws, aq_out=b.aq[0], as_out=b.as_[0],
                                             x_out=xs[xo][0], y_out=b.y[0], logits_out=b.glog[0], next_qkv=nxt,
                                             next_attn=nat)
                else:
                    call = FusedRouterLayerCall(xs[cur][0], b.oproj[0], lw.post_norm, c.rms_eps, lw.gate.wp,
                                                lw.gate.ws, c.top_k, lw.experts, b.moe[0], self.layer_ws,
                                                x_out=xs[xo][0], y_out=b.y[0], logits_out=b.glog[0], next_qkv=nxt)
                self._fr_calls[("tail", l)] = call
            call(s)
            if on_layer is not None:
                on_layer(l, xs[xo], b.moe)
            if l + 1 < L:
                cur = xn
        return xs[xo], xs[xn]

    def run(self, on_layer=None):
        """Issue one step on the current stream.  on_layer(l, x, moe): an
        optional eager hook after each layer's MoE (x is the residual stream
        before the MoE residual is added)."""
        lib, c, b, M = self.lib, self.cfg, self.b, self.M
        s = torch.cuda.current_stream().cuda_stream
        H, D, Hq, Hkv = c.hidden, c.head_dim, c.n_heads, c.n_kv_heads
        m = self.model
        self._ck(lib.mxfp4_embed_rows(m.embed.wp.data_ptr(), m.embed.ws.data_ptr(), c.vocab, H, b.ids.data_ptr(), M,
                                      b.x.data_ptr(), s), "embed_rows")
        xa, xb = b.x, b.x2          # residual stream ping-pong
        if self.qkv_tail:
            xa, xb = self._layers_qkv_tail(on_layer, s)
        for l, lw in enumerate(m.layers if not self.qkv_tail else ()):
            # input norm (+ the previous layer's MoE residual) and the q|k|v projection
            resid = b.moe if l > 0 else None
            self._norm_lin(xa, resid, lw.in_norm, xb if l > 0 else None, False, lw.qkv, b.qkv, s)
            if l > 0:
                xa, xb = xb, xa
            self._attn_oproj(l, lw, b.qkv, s)
            if self.fused_router:
                # x = x + bf16(o), its RMSNorm (y), the router logits and the MoE in one launch
                key = (l, xa.data_ptr())
                call = self._fr_calls.get(key)
                if call is None:
                    call = FusedRouterLayerCall(xa[0], b.oproj[0], lw.post_norm, c.rms_eps, lw.gate.wp, lw.gate.ws,
                                                c.top_k, lw.experts, b.moe[0], self.layer_ws, x_out=xb[0],
                                                y_out=b.y[0], logits_out=b.glog[0])
                    self._fr_calls[key] = call
                call(s)
                xa, xb = xb, xa
            else:
                # x = x + bf16(o); post-attention norm (y, MXFP4 rows for the MoE); router logits
                self._norm_lin(xa, b.oproj, lw.post_norm, xb, True, lw.gate, b.glog, s)
                xa, xb = xb, xa
                # MoE
                if M == 1:
                    self.moe_calls[l](s)
                else:
                    self._moe_batch(lw.experts, s)
            if on_layer is not None:
                on_layer(l, xa, b.moe)
        # final norm (+ the last MoE residual), lm_head, greedy next tokens
        self._ck(lib.mxfp4_rmsnorm_quant(xa.data_ptr(), b.moe.data_ptr(), m.final_norm.data_ptr(), c.rms_eps, M, H,
                                         xb.data_ptr(), b.y.data_ptr(), b.yq.data_ptr(), b.ys.data_ptr(), s),
                 "rmsnorm_quant")
        self._lin(b.yq, b.ys, m.lm_head, c.vocab, H, b.logits, s)
        self._ck(lib.mxfp4_argmax_advance(b.logits.data_ptr(), M, c.vocab, b.ids.data_ptr(), b.dpos.data_ptr(),
                                          b.arg_ws.data_ptr(), b.arg_ws.numel(), s), "argmax_advance")
        self.x_final = xb

    def _moe_batch(self, ex, s):
        lib, c, b, M = self.lib, self.cfg, self.b, self.M
        E, H, Mi = c.top_k, c.hidden, c.moe_inter
        self._ck(lib.mxfp4_route_topk(b.glog.data_ptr(), c.n_experts, M, c.n_experts, E, 1, b.rid.data_ptr(), None,
                                      b.rw.data_ptr(), s), "route_topk")
        self._ck(lib.mxfp4_moe_decode_batch(b.yq.data_ptr(), b.ys.data_ptr(), b.rid.data_ptr(), b.rw.data_ptr(),
                                            ex.gate_wp.data_ptr(), ex.gate_ws.data_ptr(), ex.up_wp.data_ptr(),
                                            ex.up_ws.data_ptr(), ex.down_wp.data_ptr(), ex.down_ws.data_ptr(),
                                            c.n_experts, M, E, H, Mi, b.moe.data_ptr(), b.moe_ws.data_ptr(),
                                            b.moe_ws.numel(), s), "moe_decode_batch")

    def check_status(self):
        """Raise if a fused MoE layer of the steps issued so far (eager or
        graph replays) reported an expired bounded wait.  Its output is then
        garbage: the down workgroups that stopped waiting never wrote their
        columns, so the step would add a stale MoE output.  The workspace is
        re-initialised before raising, as the fused layer's contract asks.
        Synchronises the device (reads the flag)."""
        if self.M != 1:
            return   # the batched MoE (route_topk + moe_decode_batch) has no cross-workgroup waits
        torch.cuda.synchronize()
        flag = layer_status(self.layer_ws)
        if flag != 0:
            c = self.cfg
            _lib.check(self.lib.mxfp4_decode_layer_reset(self.layer_ws.data_ptr(), c.top_k, c.hidden, c.moe_inter,
                                                         torch.cuda.current_stream().cuda_stream),
                       "decode_layer_reset")
            torch.cuda.synchronize()
            raise RuntimeError(f"decode step: a fused MoE layer's bounded wait expired (flag {flag}); "
                               "the step's outputs are invalid (workspace re-initialised)")

    def run_moe_only(self):
        """The step's 48 MoE blocks alone, on the buffers the last step left
        (router logits, normed activations): for measuring the MoE share."""
        s = torch.cuda.current_stream().cuda_stream
        for l, lw in enumerate(self.model.layers):
            if self.M == 1:
                self.moe_calls[l](s)
            else:
                self._moe_batch(lw.experts, s)

    def capture_fn(self, fn):
        """Any issue function captured in a HIP graph (fn runs once first)."""
        fn()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                fn()
        torch.cuda.synchronize()
        return graph

    # ------------------------------------------------------------------ graphs
    def capture(self):
        """One step captured in a HIP graph (replay = one more step)."""
        self.run()                       # warm-up (also advances the state)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                self.run()
        torch.cuda.synchronize()
        return graph
