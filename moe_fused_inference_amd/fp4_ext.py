"""Drop-in counterpart of the reference's extension loader (runtime/fp4_ext.py).

``get_ext()`` returns the ``mxfp4_linear_ext`` surface (``forward``) and
``get_decode_ext()`` the ``mxfp4_decode_ext`` surface (``prequant``,
``lin_pq``, ``moe_gateup``, ``moe_down``, ``moe_combine``, ``moe_gateup_tab``,
``moe_down_tab``, ``attn_decode`` and ``kv_write``).
Names, argument order, argument meaning, output shapes/dtypes and the
argument checks (RuntimeError with the reference's messages) follow the
pybind bindings src/ext/mxfp4_binding.cpp:21-50 and
src/ext/mxfp4_decode_binding.cpp:44-243.  Underneath, every op is one or
two calls into the C ABI of include/mxfp4_hip.h (libmxfp4_hip.so, gfx950),
launched on torch's current HIP stream; outputs are allocated with torch's
caching allocator on the input's device, as the reference does.

Two bindings carry that surface:
  * ``binding="compiled"`` (the default, as the reference's loaders return
    compiled pybind modules): the submodules ``linear`` and ``decode`` of
    ``lib/mxfp4_ext.so``, built by ``build.py`` from ``csrc/torch_binding.cpp``;
  * ``binding="ctypes"``: the Python classes below, over ctypes.
Both check the same arguments with the same messages and make the same
C-ABI calls, so their outputs are bit-identical; they differ in host time
per call.  Neither has a fallback: a missing library raises ImportError.
"""
import importlib.util
import os

import torch

from . import _lib

EXT_PATH = os.path.join(os.path.dirname(_lib.LIB_PATH), "mxfp4_ext.so")

_DT = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _ptr_table(ts):
    """Host pointer table (src/ext/mxfp4_decode_binding.cpp:44-60 checks)."""
    _require(len(ts) > 0, "empty pointer table")
    ptrs = []
    for t in ts:
        _require(t.is_cuda and t.dtype == torch.uint8, "ptr table entries must be cuda uint8")
        ptrs.append(t.data_ptr())
    return _lib.ptr_array(ptrs)


class LinearExt:
    """``mxfp4_linear_ext`` (src/ext/mxfp4_binding.cpp:47-50)."""

    __name__ = "mxfp4_linear_ext"

    def __init__(self):
        self._lib = _lib.load()

    def forward(self, x, wp, wsc):
        """x (M,K) half|bf16, wp (N,Kp/2) u8, wsc (N,Kp/32) u8 -> f32 (M,N).
        Activations are rounded to fp16 then MXFP4-quantized per 32-block
        (src/ext/mxfp4_binding.cpp:21-45)."""
        _require(x.is_cuda, "x must be cuda")
        _require(wp.is_cuda and wsc.is_cuda, "weights must be cuda")
        _require(wp.dtype == torch.uint8 and wsc.dtype == torch.uint8, "weight tensors must be uint8")
        xh = x if x.dtype in (torch.float16, torch.bfloat16) else x.to(torch.float16)
        xh = xh.contiguous()
        wp = wp.contiguous()
        wsc = wsc.contiguous()
        M, K = x.shape[0], x.shape[1]
        N, Kp = wp.shape[0], wp.shape[1] * 2
        y = torch.empty((M, N), dtype=torch.float32, device=x.device)
        if M == 0 or N == 0:
            return y
        wsb = self._lib.mxfp4_linear_workspace_size(M, Kp)
        ws = torch.empty(wsb + 256, dtype=torch.uint8, device=x.device)
        base = ws.data_ptr()
        aligned = (base + 255) & ~255
        _lib.check(self._lib.mxfp4_linear_forward(
            xh.data_ptr(), _DT[xh.dtype], wp.data_ptr(), wsc.data_ptr(), y.data_ptr(),
            M, N, K, Kp, aligned, wsb, _stream(x)), "forward")
        return y


class DecodeExt:
    """``mxfp4_decode_ext`` (src/ext/mxfp4_decode_binding.cpp:232-243)."""

    __name__ = "mxfp4_decode_ext"

    def __init__(self):
        self._lib = _lib.load()

    def prequant(self, x):
        """x (M,K) bf16 cuda -> [xq (M,Kp/2) u8, xsc (M,Kp/32) u8], Kp = ceil32(K)."""
        _require(x.is_cuda, "x must be cuda")
        _require(x.dtype == torch.bfloat16, "x must be bfloat16")
        x = x.contiguous()
        M, K = int(x.shape[0]), int(x.shape[1])
        Kp = (K + 31) // 32 * 32
        xq = torch.empty((M, Kp // 2), dtype=torch.uint8, device=x.device)
        xsc = torch.empty((M, Kp // 32), dtype=torch.uint8, device=x.device)
        if M and Kp:
            _lib.check(self._lib.mxfp4_prequant(x.data_ptr(), K, M, K, Kp, xq.data_ptr(),
                                                xsc.data_ptr(), _stream(x)), "prequant")
        return [xq, xsc]

    def lin_pq(self, xq, xsc, wp, wsc, M, N, K):
        """Pre-quantized static linear -> f32 (M,N); Kp = 2*wp.size(1)."""
        xq, xsc, wp, wsc = xq.contiguous(), xsc.contiguous(), wp.contiguous(), wsc.contiguous()
        M, N, K = int(M), int(N), int(K)
        Kp = int(wp.shape[1]) * 2
        y = torch.empty((M, N), dtype=torch.float32, device=xq.device)
        _lib.check(self._lib.mxfp4_lin_pq(xq.data_ptr(), xsc.data_ptr(), wp.data_ptr(), wsc.data_ptr(),
                                          y.data_ptr(), M, N, K, Kp, _stream(xq)), "lin_pq")
        return y

    def moe_gateup(self, xq, xsc, wps, wscs, E, M, N, K):
        """Grouped gate+up over a token-major table of 2E*M weights -> f32 (M*E, 2N)."""
        E, M, N, K = int(E), int(M), int(N), int(K)
        _require(len(wps) == 2 * E * M, "wps must be 2E*M")
        _require(len(wscs) == 2 * E * M, "wscs must be 2E*M")
        Kp = int(wps[0].shape[1]) * 2
        tw, ts = _ptr_table(wps), _ptr_table(wscs)
        gu = torch.empty((M * E, 2 * N), dtype=torch.float32, device=xq.device)
        _lib.check(self._lib.mxfp4_moe_gateup(xq.data_ptr(), xsc.data_ptr(), tw, ts, gu.data_ptr(),
                                              E, M, N, K, Kp, _stream(xq)), "moe_gateup")
        return gu

    def moe_down(self, gu, wps, wscs, E, M, N, K):
        """Fused silu(gate)*up -> MXFP4 -> down over E*M weights -> f32 (M*E, N)."""
        E, M, N, K = int(E), int(M), int(N), int(K)
        _require(len(wps) == E * M, "wps must be E*M")
        Kp = int(wps[0].shape[1]) * 2
        _require(gu.shape[0] == M * E and gu.shape[1] == 2 * K, "gu (M*E,2K)")
        tw, ts = _ptr_table(wps), _ptr_table(wscs)
        gu = gu.contiguous()
        yd = torch.empty((M * E, N), dtype=gu.dtype, device=gu.device)
        _lib.check(self._lib.mxfp4_moe_down(gu.data_ptr(), tw, ts, yd.data_ptr(), E, M, N, K, Kp,
                                            _stream(gu)), "moe_down")
        return yd

    def moe_combine(self, yd, w, M):
        """out[m,c] = sum_{e<min(E,8)} w[m,e]*yd[m*E+e,c] -> f32 (M,N); E = w.numel()/M."""
        yd, w = yd.contiguous(), w.contiguous()
        M = int(M)
        _require(M > 0, "w (M,E)")
        E = int(w.numel()) // M
        N = int(yd.shape[1])
        _require(M * E == w.numel(), "w (M,E)")
        _require(yd.shape[0] == M * E, "yd (M*E,N)")
        out = torch.empty((M, N), dtype=yd.dtype, device=yd.device)
        _lib.check(self._lib.mxfp4_moe_combine(yd.data_ptr(), N, w.data_ptr(), E, out.data_ptr(), M, N,
                                               _stream(yd)), "moe_combine")
        return out

    def moe_gateup_tab(self, xq, xsc, wps_tab, wscs_tab, E, M, N, K):
        """moe_gateup with device int64 pointer tables; Kp = 2*xq.size(1)."""
        E, M, N, K = int(E), int(M), int(N), int(K)
        Kp = int(xq.shape[1]) * 2
        gu = torch.empty((M * E, 2 * N), dtype=torch.float32, device=xq.device)
        _lib.check(self._lib.mxfp4_moe_gateup_devtab(xq.data_ptr(), xsc.data_ptr(), wps_tab.data_ptr(),
                                                     wscs_tab.data_ptr(), gu.data_ptr(), E, M, N, K, Kp,
                                                     _stream(xq)), "moe_gateup_tab")
        return gu

    def moe_down_tab(self, gu, wps_tab, wscs_tab, E, M, N, K):
        """moe_down with device int64 pointer tables; Kp = ceil32(gu.size(1)/2)."""
        E, M, N, K = int(E), int(M), int(N), int(K)
        Kp = ((int(gu.shape[1]) // 2) + 31) // 32 * 32
        yd = torch.empty((M * E, N), dtype=gu.dtype, device=gu.device)
        _lib.check(self._lib.mxfp4_moe_down_devtab(gu.data_ptr(), wps_tab.data_ptr(), wscs_tab.data_ptr(),
                                                   yd.data_ptr(), E, M, N, K, Kp, _stream(gu)), "moe_down_tab")
        return yd

    def attn_decode(self, q, kvk, kvv, dpos, sc, M):
        """Decode attention over one layer's E4M3 KV cache -> f32 (M,Hq,D).

        q (M,Hq,D) bf16; kvk/kvv (max_pos,Hkv,D) u8; dpos (1,) int32 on the
        device (base position; token m attends to 0..dpos+m); sc
        (M,Hq,max_pos) f32 scratch that receives the raw scores
        (src/ext/mxfp4_decode_binding.cpp:213-230)."""
        _require(torch.is_tensor(q) and q.dim() == 3 and q.dtype == torch.bfloat16 and q.is_cuda,
                 "q must be a cuda bf16 (M,Hq,D) tensor")
        q = q.contiguous()
        M = int(M)
        _require(kvk.dtype == torch.uint8 and kvv.dtype == torch.uint8 and kvk.dim() == 3 and kvv.shape == kvk.shape,
                 "kvk/kvv must be uint8 (max_pos,Hkv,D) tensors of one shape")
        _require(kvk.is_contiguous() and kvv.is_contiguous(), "kvk/kvv must be contiguous")
        _require(dpos.dtype == torch.int32 and dpos.is_cuda, "dpos must be a cuda int32 tensor")
        Hq, D = int(q.shape[1]), int(q.shape[2])
        max_pos, Hkv = int(kvk.shape[0]), int(kvk.shape[1])
        _require(int(q.shape[0]) >= M, "q has fewer than M rows")
        _require(sc.dtype == torch.float32 and sc.is_contiguous() and sc.numel() >= M * Hq * max_pos,
                 "sc must be a contiguous f32 buffer of M*Hq*max_pos elements")
        o = torch.empty((M, Hq, D), dtype=torch.float32, device=q.device)
        wsb = self._lib.mxfp4_attn_decode_workspace_size(M, Hq, max_pos)
        ws = torch.empty(wsb, dtype=torch.uint8, device=q.device)
        _lib.check(self._lib.mxfp4_attn_decode(q.data_ptr(), kvk.data_ptr(), kvv.data_ptr(), dpos.data_ptr(),
                                               sc.data_ptr(), o.data_ptr(), M, Hq, Hkv, D, max_pos, ws.data_ptr(),
                                               wsb, _stream(q)), "attn_decode")
        return o

    def kv_write(self, k, v, kvk, kvv, dpos, M):
        """k/v (M,Hkv,D) bf16 -> E4M3 bytes at rows dpos+m of kvk/kvv
        (max_pos,Hkv,D) u8, in place (src/ext/mxfp4_decode_binding.cpp:161-173)."""
        _require(torch.is_tensor(k) and torch.is_tensor(v) and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
                 and k.is_cuda and v.is_cuda, "k/v must be cuda bf16")
        k, v = k.contiguous(), v.contiguous()
        M = int(M)
        _require(kvk.dtype == torch.uint8 and kvv.dtype == torch.uint8 and kvk.dim() == 3 and kvv.shape == kvk.shape,
                 "kvk/kvv must be uint8 (max_pos,Hkv,D) tensors of one shape")
        _require(kvk.is_contiguous() and kvv.is_contiguous(), "kvk/kvv must be contiguous")
        _require(dpos.dtype == torch.int32 and dpos.is_cuda, "dpos must be a cuda int32 tensor")
        max_pos, Hkv, D = (int(d) for d in kvk.shape)
        _require(k.numel() >= M * Hkv * D and v.numel() >= M * Hkv * D, "k/v have fewer than M*Hkv*D elements")
        _lib.check(self._lib.mxfp4_kv_write(k.data_ptr(), v.data_ptr(), kvk.data_ptr(), kvv.data_ptr(),
                                            dpos.data_ptr(), M, Hkv, D, max_pos, _stream(k)), "kv_write")


_compiled = None
_ctypes = {}


def load_compiled():
    """The compiled binding module (once).  Raises ImportError if it is not built."""
    global _compiled
    if _compiled is None:
        _lib.load()
        if not os.path.exists(EXT_PATH):
            raise ImportError(
                f"moe_fused_inference_amd: torch binding not built ({EXT_PATH}); "
                "run `python -m moe_fused_inference_amd.build` (or __graft_entry__.build())")
        spec = importlib.util.spec_from_file_location("mxfp4_ext", EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _compiled = mod
    return _compiled


def _get(binding, sub, cls):
    if binding == "compiled":
        return getattr(load_compiled(), sub)
    if binding == "ctypes":
        if cls not in _ctypes:
            _ctypes[cls] = cls()
        return _ctypes[cls]
    raise ValueError(f"binding must be 'compiled' or 'ctypes', got {binding!r}")


def get_ext(binding="compiled"):
    """Counterpart of runtime/fp4_ext.py:21-39 (module ``mxfp4_linear_ext``)."""
    return _get(binding, "linear", LinearExt)


def get_decode_ext(binding="compiled"):
    """Counterpart of runtime/fp4_ext.py:46-62 (module ``mxfp4_decode_ext``)."""
    return _get(binding, "decode", DecodeExt)
