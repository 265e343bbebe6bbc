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
