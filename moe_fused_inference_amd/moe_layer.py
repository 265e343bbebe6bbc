"""Fused decode MoE layer on stacked per-layer expert weights.

A layer's experts are kept resident in HBM as six stacked tensors whose
per-expert slices are byte-identical to the reference's packed tensors
(quant/quantize_mxfp4.py:145-159, runtime/weight_store.py:278-284):
    gate_wp / up_wp   (n_experts, Mi, H/2) u8     gate_ws / up_ws  (n_experts, Mi, H/32) u8
    down_wp           (n_experts, H, Mi/2) u8     down_ws          (n_experts, H, Mi/32) u8
``decode_layer`` runs one token through the layer with a single HIP launch
(mxfp4_moe_decode_layer in include/mxfp4_hip.h).
"""
import ctypes
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class StackedExperts:
    gate_wp: torch.Tensor
    gate_ws: torch.Tensor
    up_wp: torch.Tensor
    up_ws: torch.Tensor
    down_wp: torch.Tensor
    down_ws: torch.Tensor

    @property
    def n_experts(self):
        return int(self.gate_wp.shape[0])

    @property
    def hidden(self):
        return int(self.gate_wp.shape[2]) * 2

    @property
    def inter(self):
        return int(self.gate_wp.shape[1])

    def expert(self, e):
        """Spec dicts of expert e in the reference's layout ({'wp','wsc','K'})."""
        return {"gate": {"wp": self.gate_wp[e], "wsc": self.gate_ws[e], "K": self.hidden},
                "up": {"wp": self.up_wp[e], "wsc": self.up_ws[e], "K": self.hidden},
                "down": {"wp": self.down_wp[e], "wsc": self.down_ws[e], "K": self.inter}}

    def check(self):
        n, Mi, H = self.n_experts, self.inter, self.hidden
        shapes = {"gate_wp": (n, Mi, H // 2), "gate_ws": (n, Mi, H // 32), "up_wp": (n, Mi, H // 2),
                  "up_ws": (n, Mi, H // 32), "down_wp": (n, H, Mi // 2), "down_ws": (n, H, Mi // 32)}
        for k, shp in shapes.items():
            t = getattr(self, k)
            if tuple(t.shape) != shp or t.dtype != torch.uint8 or not t.is_cuda or not t.is_contiguous():
                raise RuntimeError(f"{k} must be a contiguous cuda uint8 tensor of shape {shp}")


def workspace(E, Mi, H=2048, device="cuda"):
    """Workspace for decode_layer launches of shape (E, H, Mi), initialised on
    the current stream.  Launches sharing it must be stream-ordered."""
    lib = _lib.load()
    n = lib.mxfp4_decode_layer_workspace_size(E, Mi)
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    _lib.check(lib.mxfp4_decode_layer_reset(ws.data_ptr(), E, H, Mi, torch.cuda.current_stream().cuda_stream),
               "decode_layer_reset")
    return ws


class DecodeLayerCall:
    """Pre-bound arguments of one fused-layer launch (cheap to re-issue and
    to capture in a HIP graph: routing travels by value in the kernel
    arguments, or from device tensors)."""

    def __init__(self, x, ids, w, experts, out, resid, ws):
        self.lib = _lib.load()
        E = len(ids) if not torch.is_tensor(ids) else int(ids.numel())
        dev_routing = torch.is_tensor(ids) and ids.is_cuda
        if dev_routing:
            if ids.dtype != torch.int32 or w.dtype != torch.float32 or not w.is_cuda:
                raise RuntimeError("device routing must be int32 ids and float32 weights on the GPU")
            self.ids_h = self.w_h = None
            ids_d, w_d = ids.data_ptr(), w.data_ptr()
        else:
            self.ids_h = (ctypes.c_int32 * E)(*[int(i) for i in ids])
            self.w_h = (ctypes.c_float * E)(*[float(v) for v in w])
            ids_d = w_d = None
        self.keep = (x, ids, w, experts, out, resid, ws)
        self.args = (x.data_ptr(), self.ids_h, self.w_h, ids_d, w_d,
                     experts.gate_wp.data_ptr(), experts.gate_ws.data_ptr(),
                     experts.up_wp.data_ptr(), experts.up_ws.data_ptr(),
                     experts.down_wp.data_ptr(), experts.down_ws.data_ptr(),
                     experts.n_experts, E, experts.hidden, experts.inter,
                     out.data_ptr(), resid.data_ptr() if resid is not None else None,
                     ws.data_ptr(), ws.numel())

    def __call__(self, stream=None):
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _lib.check(self.lib.mxfp4_moe_decode_layer(*self.args, s), "moe_decode_layer")


class RoutedLayerCall:
    """Pre-bound arguments of one fused-layer launch that routes itself from
    the layer's fp32 router logits (mxfp4_moe_decode_layer_routed)."""

    def __init__(self, x, logits, E, experts, out, resid, ws, norm=True, ids_out=None, w_out=None):
        self.lib = _lib.load()
        if logits.dtype != torch.float32 or not logits.is_cuda or not logits.is_contiguous():
            raise RuntimeError("logits must be a contiguous cuda float32 tensor")
        if logits.numel() != experts.n_experts:
            raise RuntimeError(f"logits has {logits.numel()} entries, expected n_experts={experts.n_experts}")
        if (ids_out is None) != (w_out is None):
            raise RuntimeError("give ids_out and w_out both or neither")
        self.keep = (x, logits, experts, out, resid, ws, ids_out, w_out)
        self.args = (x.data_ptr(), logits.data_ptr(), int(bool(norm)),
                     ids_out.data_ptr() if ids_out is not None else None,
                     w_out.data_ptr() if w_out is not None else None,
                     experts.gate_wp.data_ptr(), experts.gate_ws.data_ptr(),
                     experts.up_wp.data_ptr(), experts.up_ws.data_ptr(),
                     experts.down_wp.data_ptr(), experts.down_ws.data_ptr(),
                     experts.n_experts, int(E), experts.hidden, experts.inter,
                     out.data_ptr(), resid.data_ptr() if resid is not None else None,
                     ws.data_ptr(), ws.numel())

    def __call__(self, stream=None):
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _lib.check(self.lib.mxfp4_moe_decode_layer_routed(*self.args, s), "moe_decode_layer_routed")


class FusedRouterLayerCall:
    """Pre-bound arguments of one fused-layer launch that also runs the
    post-attention residual add, RMSNorm and router projection
    (mxfp4_moe_decode_layer_fused_router): x bf16 (H,) and resid fp32 (H,)
    in, x_out = bf16(x + bf16(resid)), the MoE of h2 = rms_norm(x_out) * norm_w
    in `out` (fp32 (H,)), routed on the logits of the MXFP4 router
    (router_wp, router_ws) computed in the same launch.

    With next_qkv = (norm_w, wp, ws, qkv_out[, x_next]) the launch also runs
    the next layer's input residual, RMSNorm and q|k|v projection
    (mxfp4_moe_decode_layer_fused_router_qkv): x_next = bf16(x_out +
    bf16(out)), qkv_out fp32 (Nq,) = MXFP4(rms_norm(x_next) * norm_w) . W^T
    for the MXFP4 W = (wp (Nq, H/2), ws (Nq, H/32)); x_next must not alias x or x_out."""

    def __init__(self, x, resid, norm_w, eps, router_wp, router_ws, E, experts, out, ws, norm=True, x_out=None,
                 y_out=None, logits_out=None, ids_out=None, w_out=None, next_qkv=None):
        self.lib = _lib.load()
        if (ids_out is None) != (w_out is None):
            raise RuntimeError("give ids_out and w_out both or neither")
        n, H = experts.n_experts, experts.hidden
        if tuple(router_wp.shape) != (n, H // 2) or tuple(router_ws.shape) != (n, H // 32):
            raise RuntimeError(f"router weights must be ({n}, {H // 2}) + ({n}, {H // 32})")
        if resid.dtype != torch.float32 or x.dtype != torch.bfloat16 or norm_w.dtype != torch.bfloat16:
            raise RuntimeError("x and norm_w must be bfloat16, resid float32")
        ptr = (lambda t: t.data_ptr() if t is not None else None)
        self.keep = (x, resid, norm_w, router_wp, router_ws, experts, out, ws, x_out, y_out, logits_out, ids_out,
                     w_out, next_qkv)
        head = (x.data_ptr(), resid.data_ptr(), norm_w.data_ptr(), float(eps), router_wp.data_ptr(),
                router_ws.data_ptr(), int(bool(norm)), ptr(x_out), ptr(y_out), ptr(logits_out), ptr(ids_out),
                ptr(w_out), experts.gate_wp.data_ptr(), experts.gate_ws.data_ptr(),
                experts.up_wp.data_ptr(), experts.up_ws.data_ptr(),
                experts.down_wp.data_ptr(), experts.down_ws.data_ptr(),
                n, int(E), H, experts.inter)
        tail = (out.data_ptr(), ws.data_ptr(), ws.numel())
        if next_qkv is None:
            self.fn, self.what = self.lib.mxfp4_moe_decode_layer_fused_router, "moe_decode_layer_fused_router"
            self.args = head + tail
        else:
            qnw, qwp, qws, qkv_out = next_qkv[:4]
            x_next = next_qkv[4] if len(next_qkv) > 4 else None
            nq = qwp.shape[0]
            if tuple(qwp.shape) != (nq, H // 2) or tuple(qws.shape) != (nq, H // 32) or qwp.dtype != torch.uint8:
                raise RuntimeError(f"q|k|v weights must be uint8 (Nq, {H // 2}) + (Nq, {H // 32})")
            if qkv_out.dtype != torch.float32 or qkv_out.numel() != nq or qnw.dtype != torch.bfloat16:
                raise RuntimeError("qkv_out must be float32 (Nq,), the norm weight bfloat16")
            if x_next is not None and x_next.data_ptr() in (x.data_ptr(), ptr(x_out)):
                raise RuntimeError("x_next must not alias x or x_out")
            self.fn, self.what = self.lib.mxfp4_moe_decode_layer_fused_router_qkv, "moe_decode_layer_fused_router_qkv"
            self.args = head + (qnw.data_ptr(), qwp.data_ptr(), qws.data_ptr(), nq, qkv_out.data_ptr(),
                                ptr(x_next)) + tail

    def __call__(self, stream=None):
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _lib.check(self.fn(*self.args, s), self.what)


class PostAttnLayerCall:
    """Pre-bound arguments of mxfp4_decode_layer_post_attn: the merge of the
    token's attention chunk records (attn_ws, as mxfp4_attn_decode_fused_partials
    left it for max_pos positions, dpos the position on the device), o_proj
    (o_wp uint8 (H, 2048), o_ws uint8 (H, 128): 32 heads of 128) into
    oproj_out fp32 (H,), then the fused-router MoE launch of
    FusedRouterLayerCall on (x, oproj_out), with the same optional outputs
    and next_qkv tail; aq_out / as_out optionally receive the attention
    output's MXFP4 row.  next_attn = (attn_ws_next, kvk_next, kvv_next,
    q_norm_next, k_norm_next, Hkv, theta, codec), with next_qkv: the next
    layer's attention chunk pass in the same launch, on next_qkv's output,
    leaving its records in attn_ws_next (a buffer other than attn_ws)."""

    def __init__(self, attn_ws, dpos, max_pos, o_wp, o_ws, oproj_out, x, norm_w, eps, router_wp, router_ws, E,
                 experts, out, ws, norm=True, aq_out=None, as_out=None, x_out=None, y_out=None, logits_out=None,
                 ids_out=None, w_out=None, next_qkv=None, next_attn=None):
        self.lib = _lib.load()
        n, H = experts.n_experts, experts.hidden
        hq = 32
        if tuple(o_wp.shape) != (H, hq * 64) or tuple(o_ws.shape) != (H, hq * 4):
            raise RuntimeError(f"o_proj weights must be ({H}, {hq * 64}) + ({H}, {hq * 4})")
        if (aq_out is None) != (as_out is None):
            raise RuntimeError("give aq_out and as_out both or neither")
        if oproj_out.dtype != torch.float32 or oproj_out.numel() != H:
            raise RuntimeError("oproj_out must be float32 (H,)")
        ptr = (lambda t: t.data_ptr() if t is not None else None)
        if next_qkv is None:
            qkv = (None, None, None, 0, None, None)
        else:
            qnw, qwp, qws, qkv_out = next_qkv[:4]
            x_next = next_qkv[4] if len(next_qkv) > 4 else None
            nq = qwp.shape[0]
            if tuple(qwp.shape) != (nq, H // 2) or tuple(qws.shape) != (nq, H // 32) or qkv_out.numel() != nq:
                raise RuntimeError("q|k|v weights must be (Nq, H/2) + (Nq, H/32), qkv_out (Nq,)")
            qkv = (qnw.data_ptr(), qwp.data_ptr(), qws.data_ptr(), nq, qkv_out.data_ptr(), ptr(x_next))
        if next_attn is None:
            nat = (None, 0, None, None, None, None, 0, 0.0, 0)
        else:
            aws_n, kvk_n, kvv_n, qn_n, kn_n, hkv, theta, codec = next_attn
            nat = (aws_n.data_ptr(), aws_n.numel() * aws_n.element_size(), kvk_n.data_ptr(), kvv_n.data_ptr(),
                   qn_n.data_ptr(), kn_n.data_ptr(), int(hkv), float(theta), int(codec))
        self.keep = (attn_ws, dpos, o_wp, o_ws, oproj_out, x, norm_w, router_wp, router_ws, experts, out, ws, aq_out,
                     as_out, x_out, y_out, logits_out, ids_out, w_out, next_qkv, next_attn)
        self.args = ((attn_ws.data_ptr(), attn_ws.numel() * attn_ws.element_size(), dpos.data_ptr(), hq,
                      int(max_pos), ptr(aq_out), ptr(as_out), o_wp.data_ptr(), o_ws.data_ptr(),
                      oproj_out.data_ptr(), x.data_ptr(), norm_w.data_ptr(), float(eps), router_wp.data_ptr(),
                      router_ws.data_ptr(), int(bool(norm)), ptr(x_out), ptr(y_out), ptr(logits_out), ptr(ids_out),
                      ptr(w_out), experts.gate_wp.data_ptr(), experts.gate_ws.data_ptr(), experts.up_wp.data_ptr(),
                      experts.up_ws.data_ptr(), experts.down_wp.data_ptr(), experts.down_ws.data_ptr(), n, int(E),
                      H, experts.inter) + qkv + nat + (out.data_ptr(), ws.data_ptr(), ws.numel()))

    def __call__(self, stream=None):
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _lib.check(self.lib.mxfp4_decode_layer_post_attn(*self.args, s), "decode_layer_post_attn")


def decode_layer_routed(x, logits, E, experts, norm=True, out=None, resid=None, ws=None, want_routing=False):
    """One token through the layer, routing included: softmax / top-E /
    renormalise of the fp32 router logits (n_experts,) computed in the same
    launch.  Returns (out, resid) or, with want_routing, (out, resid, ids
    int32 (E,), w fp32 (E,))."""
    experts.check()
    if x.dtype != torch.bfloat16 or not x.is_cuda:
        raise RuntimeError("x must be a cuda bfloat16 tensor")
    x = x.reshape(-1).contiguous()
    logits = logits.reshape(-1).float().contiguous()
    if out is None:
        out = torch.empty(experts.hidden, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = workspace(E, experts.inter, experts.hidden, x.device)
    ids = torch.empty(E, dtype=torch.int32, device=x.device) if want_routing else None
    w = torch.empty(E, dtype=torch.float32, device=x.device) if want_routing else None
    RoutedLayerCall(x, logits, E, experts, out, resid, ws, norm, ids, w)()
    return (out, resid, ids, w) if want_routing else (out, resid)


def decode_layer(x, ids, w, experts, out=None, resid=None, ws=None):
    """x (1, H) or (H,) bf16 -> (out fp32 (H,), resid bf16 (H,) or None).

    ids / w: the E (<= 8) routed expert ids and combine weights, as Python
    sequences (passed by value) or int32 / float32 cuda tensors."""
    experts.check()
    if x.dtype != torch.bfloat16 or not x.is_cuda:
        raise RuntimeError("x must be a cuda bfloat16 tensor")
    x = x.reshape(-1).contiguous()
    if x.numel() != experts.hidden:
        raise RuntimeError(f"x has {x.numel()} elements, expected H={experts.hidden}")
    E = len(ids) if not torch.is_tensor(ids) else int(ids.numel())
    if out is None:
        out = torch.empty(experts.hidden, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = workspace(E, experts.inter, experts.hidden, x.device)
    DecodeLayerCall(x, ids, w, experts, out, resid, ws)()
    return out, resid


def layer_status(ws):
    """Error flag of the fused layer's bounded wait (0 = never expired)."""
    lib = _lib.load()
    flag = ctypes.c_int(0)
    _lib.check(lib.mxfp4_decode_layer_status(ws.data_ptr(), ctypes.byref(flag)), "decode_layer_status")
    return flag.value


# ----------------------------------------------------------------------------- layer stacks
class LayerStack:
    """Consecutive MoE layers (a list of StackedExperts of one shape) for
    mxfp4_moe_decode_stack: holds the device table of each layer's six
    stacked weight pointers {gate_wp, up_wp, down_wp, gate_ws, up_ws, down_ws}."""

    def __init__(self, layers, device="cuda"):
        if not layers:
            raise RuntimeError("LayerStack needs at least one layer")
        for lay in layers:
            lay.check()
        shape = (layers[0].n_experts, layers[0].hidden, layers[0].inter)
        if any((l.n_experts, l.hidden, l.inter) != shape for l in layers):
            raise RuntimeError("all layers of a stack must have the same (n_experts, H, Mi)")
        self.layers = list(layers)
        self.n_experts, self.hidden, self.inter = shape
        rows = [[l.gate_wp.data_ptr(), l.up_wp.data_ptr(), l.down_wp.data_ptr(),
                 l.gate_ws.data_ptr(), l.up_ws.data_ptr(), l.down_ws.data_ptr()] for l in layers]
        self.table = torch.tensor(rows, dtype=torch.int64).to(device)

    def __len__(self):
        return len(self.layers)


def stack_workspace(E, H, Mi, device="cuda"):
    """Workspace for decode_stack launches of shape (E, H, Mi), initialised
    on the current stream.  Launches sharing it must be stream-ordered."""
    lib = _lib.load()
    n = lib.mxfp4_decode_stack_workspace_size(E, H, Mi)
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    _lib.check(lib.mxfp4_decode_stack_reset(ws.data_ptr(), E, H, Mi, torch.cuda.current_stream().cuda_stream),
               "decode_stack_reset")
    return ws


class DecodeStackCall:
    """Pre-bound arguments of one mxfp4_moe_decode_stack launch: x through
    every layer of `stack` with device routing ids (L, E) int32 / w (L, E)
    fp32; x_out (H,) bf16 receives x_L; x_all (L, H) bf16 and y_all (L, H)
    fp32 optionally receive every layer's x_{l+1} and moe output."""

    def __init__(self, x, ids, w, stack, x_out, ws, x_all=None, y_all=None, strict=False):
        self.lib = _lib.load()
        L = len(stack)
        if ids.dtype != torch.int32 or not ids.is_cuda or ids.dim() != 2 or ids.shape[0] != L:
            raise RuntimeError(f"ids must be a cuda int32 tensor of shape ({L}, E)")
        E = int(ids.shape[1])
        if w.dtype != torch.float32 or not w.is_cuda or tuple(w.shape) != (L, E):
            raise RuntimeError(f"w must be a cuda float32 tensor of shape ({L}, {E})")
        if not (ids.is_contiguous() and w.is_contiguous()):
            raise RuntimeError("ids and w must be contiguous")
        H = stack.hidden
        for name, t, dt, shp in (("x", x, torch.bfloat16, (H,)), ("x_out", x_out, torch.bfloat16, (H,))):
            if t.dtype != dt or not t.is_cuda or tuple(t.reshape(-1).shape) != shp or not t.is_contiguous():
                raise RuntimeError(f"{name} must be a contiguous cuda {dt} tensor of {shp[0]} elements")
        if x_all is not None and (x_all.dtype != torch.bfloat16 or tuple(x_all.shape) != (L, H)
                                  or not x_all.is_contiguous()):
            raise RuntimeError(f"x_all must be a contiguous bf16 tensor of shape ({L}, {H})")
        if y_all is not None and (y_all.dtype != torch.float32 or tuple(y_all.shape) != (L, H)
                                  or not y_all.is_contiguous()):
            raise RuntimeError(f"y_all must be a contiguous fp32 tensor of shape ({L}, {H})")
        self.keep = (x, ids, w, stack, x_out, ws, x_all, y_all)
        self.args = (x.data_ptr(), ids.data_ptr(), w.data_ptr(), stack.table.data_ptr(), L,
                     stack.n_experts, E, H, stack.inter, x_out.data_ptr(),
                     x_all.data_ptr() if x_all is not None else None,
                     y_all.data_ptr() if y_all is not None else None,
                     int(bool(strict)), ws.data_ptr(), ws.numel())

    def __call__(self, stream=None):
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _lib.check(self.lib.mxfp4_moe_decode_stack(*self.args, s), "moe_decode_stack")


def decode_stack(x, ids, w, stack, ws=None, strict=False, want_all=False):
    """x (H,) bf16 through every layer of `stack` in one launch; ids (L, E)
    int32 / w (L, E) fp32 cuda routing.  Returns x_L (H,) bf16, or with
    want_all (x_L, x_all (L, H) bf16, y_all (L, H) fp32)."""
    if x.dtype != torch.bfloat16 or not x.is_cuda:
        raise RuntimeError("x must be a cuda bfloat16 tensor")
    x = x.reshape(-1).contiguous()
    E = int(ids.shape[1])
    if ws is None:
        ws = stack_workspace(E, stack.hidden, stack.inter, x.device)
    x_out = torch.empty_like(x)
    x_all = torch.empty((len(stack), stack.hidden), dtype=torch.bfloat16, device=x.device) if want_all else None
    y_all = torch.empty((len(stack), stack.hidden), dtype=torch.float32, device=x.device) if want_all else None
    DecodeStackCall(x, ids, w, stack, x_out, ws, x_all, y_all, strict)()
    return (x_out, x_all, y_all) if want_all else x_out


def stack_status(ws):
    """Error flag of the layer stack's bounded waits (0 = never expired)."""
    lib = _lib.load()
    flag = ctypes.c_int(0)
    _lib.check(lib.mxfp4_decode_stack_status(ws.data_ptr(), ctypes.byref(flag)), "decode_stack_status")
    return flag.value


# ----------------------------------------------------------------------------- batched tokens
def moe_group(topi, n_experts):
    """GPU token->expert grouping (mxfp4_moe_group): topi (T, k) int64 ->
    (counts (n,), offsets (n,), pairs (T*k,)) int32, pairs sorted stably by
    expert id -- the order torch.where(topi == e) yields per expert
    (runtime/model_runner_v2.py:111)."""
    lib = _lib.load()
    if topi.dim() != 2 or topi.dtype != torch.int64 or not topi.is_cuda:
        raise RuntimeError("topi must be a 2-D cuda int64 tensor")
    topi = topi.contiguous()
    T, k = topi.shape
    dev = topi.device
    counts = torch.empty(n_experts, dtype=torch.int32, device=dev)
    offs = torch.empty(n_experts, dtype=torch.int32, device=dev)
    pairs = torch.full((T * k,), -1, dtype=torch.int32, device=dev)
    _lib.check(lib.mxfp4_moe_group(topi.data_ptr(), T, k, n_experts, counts.data_ptr(), offs.data_ptr(),
                                   pairs.data_ptr(), torch.cuda.current_stream(dev).cuda_stream), "moe_group")
    return counts, offs, pairs


def route_topk(logits, k, norm=True, want_int64=False, out=None):
    """GPU router top-k (mxfp4_route_topk): softmax over the last dim of the
    fp32 logits (M, n), top-k, renormalised over the winners when norm --
    runtime/model_runner_v2.py:189-192 without the host round trip.
    Returns (ids int32 (M, k), w fp32 (M, k)) and, with want_int64, also
    topi int64 (M, k) (torch.topk's dtype).  `out` = (ids, w) reuses
    preallocated contiguous tensors (e.g. bound into a captured graph)."""
    lib = _lib.load()
    if logits.dim() != 2 or logits.dtype != torch.float32 or not logits.is_cuda:
        raise RuntimeError("logits must be a 2-D cuda float32 tensor")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    M, n = logits.shape
    dev = logits.device
    if out is not None:
        ids, w = out
        if (ids.dtype != torch.int32 or w.dtype != torch.float32 or ids.numel() != M * k or w.numel() != M * k
                or not ids.is_contiguous() or not w.is_contiguous() or not ids.is_cuda or not w.is_cuda):
            raise RuntimeError(f"out must be contiguous cuda int32 / float32 tensors of {M * k} elements")
    else:
        ids = torch.empty((M, k), dtype=torch.int32, device=dev)
        w = torch.empty((M, k), dtype=torch.float32, device=dev)
    ids64 = torch.empty((M, k), dtype=torch.int64, device=dev) if want_int64 else None
    _lib.check(lib.mxfp4_route_topk(logits.data_ptr(), logits.stride(0), M, n, k, int(bool(norm)), ids.data_ptr(),
                                    ids64.data_ptr() if want_int64 else None, w.data_ptr(),
                                    torch.cuda.current_stream(dev).cuda_stream), "route_topk")
    return (ids, w, ids64) if want_int64 else (ids, w)


def route_tables(ids, experts):
    """Device pointer tables for moe_gateup_tab / moe_down_tab from device
    ids (mxfp4_route_tables): ids int32 (M, k) -> (gu_wp, gu_ws) int64
    (M*2k,) in the token-major order m*2k + proj*k + e, and (dn_wp, dn_ws)
    int64 (M*k,) -- the lists of runtime/model_runner_v2.py:279-286."""
    lib = _lib.load()
    experts.check()
    if ids.dim() != 2 or ids.dtype != torch.int32 or not ids.is_cuda:
        raise RuntimeError("ids must be a 2-D cuda int32 tensor")
    ids = ids.contiguous()
    M, k = ids.shape
    dev = ids.device
    gu_wp = torch.empty(M * 2 * k, dtype=torch.int64, device=dev)
    gu_ws = torch.empty_like(gu_wp)
    dn_wp = torch.empty(M * k, dtype=torch.int64, device=dev)
    dn_ws = torch.empty_like(dn_wp)
    _lib.check(lib.mxfp4_route_tables(ids.data_ptr(), M, k, experts.gate_wp.data_ptr(), experts.gate_ws.data_ptr(),
                                      experts.up_wp.data_ptr(), experts.up_ws.data_ptr(),
                                      experts.down_wp.data_ptr(), experts.down_ws.data_ptr(), experts.n_experts,
                                      experts.hidden, experts.inter, gu_wp.data_ptr(), gu_ws.data_ptr(),
                                      dn_wp.data_ptr(), dn_ws.data_ptr(), torch.cuda.current_stream(dev).cuda_stream),
               "route_tables")
    return gu_wp, gu_ws, dn_wp, dn_ws


def decode_batch(xq, xs, ids, w, experts, out=None, ws=None):
    """The MoE block of a batched decode step on MXFP4 activation rows
    (forward_batch's moe_gateup -> moe_down -> moe_combine,
    runtime/model_runner_v2.py:265-289) in two launches: xq (M, H/2) / xs
    (M, H/32) uint8, ids int32 (M, E), w fp32 (M, E), experts a
    StackedExperts.  Returns the fp32 (M, H) output."""
    lib = _lib.load()
    experts.check()
    M, E = ids.shape
    H, Mi = experts.hidden, experts.inter
    if xq.shape != (M, H // 2) or xs.shape != (M, H // 32) or w.shape != (M, E):
        raise RuntimeError("xq (M, H/2), xs (M, H/32), ids and w (M, E) shapes do not match")
    if ids.dtype != torch.int32 or w.dtype != torch.float32:
        raise RuntimeError("ids must be int32 and w float32")
    if out is None:
        out = torch.empty((M, H), dtype=torch.float32, device=xq.device)
    if ws is None:
        ws = torch.empty(lib.mxfp4_moe_decode_batch_workspace_size(M, E, Mi), dtype=torch.uint8, device=xq.device)
    _lib.check(lib.mxfp4_moe_decode_batch(xq.data_ptr(), xs.data_ptr(), ids.contiguous().data_ptr(),
                                          w.contiguous().data_ptr(), experts.gate_wp.data_ptr(),
                                          experts.gate_ws.data_ptr(), experts.up_wp.data_ptr(),
                                          experts.up_ws.data_ptr(), experts.down_wp.data_ptr(),
                                          experts.down_ws.data_ptr(), experts.n_experts, M, E, H, Mi,
                                          out.data_ptr(), ws.data_ptr(), ws.numel(),
                                          torch.cuda.current_stream(xq.device).cuda_stream), "moe_decode_batch")
    return out


def prefill_workspace(T, topk, n_experts, H, Mi, device="cuda"):
    """Scratch memory for one moe_compute call of this shape (reusable by
    stream-ordered calls; nothing persists between calls)."""
    lib = _lib.load()
    n = lib.mxfp4_moe_prefill_workspace_size(T, topk, n_experts, H, Mi)
    if n == 0:
        raise RuntimeError(f"invalid prefill shape T={T} topk={topk} n_experts={n_experts} H={H} Mi={Mi}")
    return torch.empty(n, dtype=torch.uint8, device=device)


def _expert_table(experts, device):
    """Reference spec dicts {e: {'gate': {'wp','wsc'}, 'up': ..., 'down': ...}}
    -> (device table (n, 6) int64, n, H, Mi, present (n,) bool)."""
    ids = sorted(int(e) for e in experts)
    n = ids[-1] + 1
    first = experts[ids[0]]
    H = int(first["gate"]["wp"].shape[1]) * 2
    Mi = int(first["gate"]["wp"].shape[0])
    tab = torch.zeros((n, 6), dtype=torch.int64)
    present = torch.zeros(n, dtype=torch.bool)
    for e in ids:
        spec = experts[e]
        for j, nm in enumerate(("gate", "up", "down")):
            wp, wsc = spec[nm]["wp"], spec[nm]["wsc"]
            want = ((Mi, H // 2), (Mi, H // 32)) if nm != "down" else ((H, Mi // 2), (H, Mi // 32))
            if (tuple(wp.shape), tuple(wsc.shape)) != want or wp.dtype != torch.uint8 or not wp.is_cuda \
                    or not wp.is_contiguous() or not wsc.is_contiguous():
                raise RuntimeError(f"expert {e} {nm}: expected contiguous cuda uint8 {want}")
            tab[e, 2 * j] = wp.data_ptr()
            tab[e, 2 * j + 1] = wsc.data_ptr()
        present[e] = True
    return tab.to(device), n, H, Mi, present.to(device)


def moe_compute(h, topi, scores, experts, out=None, ws=None):
    """Drop-in counterpart of ModelRunnerV2.moe_compute
    (runtime/model_runner_v2.py:108-122): h (T, H) bf16, topi (T, k) int64,
    scores (T, k) (used as bf16, as moe_route returns them), experts either a
    StackedExperts or the reference's dict of per-expert spec dicts.  Returns
    the bf16 (T, H) MoE output.  Five launches, no host synchronisation (the
    dict form builds a small pointer table first)."""
    lib = _lib.load()
    if h.dim() != 2 or h.dtype != torch.bfloat16 or not h.is_cuda:
        raise RuntimeError("h must be a 2-D cuda bfloat16 tensor")
    if topi.shape != scores.shape or topi.dim() != 2 or topi.shape[0] != h.shape[0]:
        raise RuntimeError("topi and scores must both be (T, k) with T = h.shape[0]")
    h = h.contiguous()
    topi = topi.to(torch.int64).contiguous()
    sc = scores.to(torch.bfloat16).contiguous()
    T, k = topi.shape
    stream = torch.cuda.current_stream(h.device).cuda_stream
    if isinstance(experts, StackedExperts):
        experts.check()
        n, H, Mi = experts.n_experts, experts.hidden, experts.inter
    else:
        tab, n, H, Mi, present = _expert_table(experts, h.device)
        # ids absent from the dict contribute nothing, as in the reference loop
        ok = (topi >= 0) & (topi < n)
        topi = torch.where(ok & present[topi.clamp(0, n - 1)], topi, torch.full_like(topi, -1))
    if h.shape[1] != H:
        raise RuntimeError(f"h has {h.shape[1]} columns, experts expect H={H}")
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=h.device)
    if ws is None:
        ws = prefill_workspace(T, k, n, H, Mi, h.device)
    if isinstance(experts, StackedExperts):
        rc = lib.mxfp4_moe_prefill(h.data_ptr(), topi.data_ptr(), sc.data_ptr(),
                                   experts.gate_wp.data_ptr(), experts.gate_ws.data_ptr(),
                                   experts.up_wp.data_ptr(), experts.up_ws.data_ptr(),
                                   experts.down_wp.data_ptr(), experts.down_ws.data_ptr(),
                                   n, T, k, H, Mi, out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "moe_prefill")
    else:
        rc = lib.mxfp4_moe_prefill_tab(h.data_ptr(), topi.data_ptr(), sc.data_ptr(), tab.data_ptr(), n, T, k, H,
                                       Mi, out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "moe_prefill_tab")
    return out
