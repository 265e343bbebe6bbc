"""ctypes binding of the C ABI in include/mxfp4_hip.h.

The library is the in-tree ``lib/libmxfp4_hip.so`` built by ``build.py``.
There is no fallback: if it is missing or does not load, importing the
operators raises, so no caller can silently run a non-HIP path.
"""
import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libmxfp4_hip.so")

_c_i = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_sz = ctypes.c_size_t

# name -> (restype, argtypes); keep in step with include/mxfp4_hip.h
SIGNATURES = {
    "mxfp4_abi_version": (_c_i, []),
    "mxfp4_selftest_wave_sum": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_p]),
    "mxfp4_last_error": (ctypes.c_char_p, []),
    "mxfp4_prequant": (_c_i, [_c_p, _c_i64, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p]),
    "mxfp4_quantize_rows": (_c_i, [_c_p, _c_i, _c_i, _c_i64, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p]),
    "mxfp4_lin_pq": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_linear_workspace_size": (_c_sz, [_c_i, _c_i]),
    "mxfp4_linear_forward": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_p, _c_sz, _c_p]),
    "mxfp4_moe_gateup": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_moe_gateup_devtab": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_moe_down": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_moe_down_devtab": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_moe_combine": (_c_i, [_c_p, _c_i, _c_p, _c_i, _c_p, _c_i, _c_i, _c_p]),
    "mxfp4_decode_layer_workspace_size": (_c_sz, [_c_i, _c_i]),
    "mxfp4_decode_layer_reset": (_c_i, [_c_p, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_decode_layer_status": (_c_i, [_c_p, ctypes.POINTER(ctypes.c_int)]),
    "mxfp4_moe_decode_layer": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                      _c_i, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_moe_decode_layer_routed": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                             _c_i, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_moe_decode_layer_fused_router": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, _c_p, _c_p, _c_i,
                                                   _c_p, _c_p, _c_p, _c_p, _c_p,
                                                   _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                                   _c_i, _c_i, _c_i, _c_i, _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_moe_decode_layer_fused_router_qkv": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, _c_p, _c_p, _c_i,
                                                       _c_p, _c_p, _c_p, _c_p, _c_p,
                                                       _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                                       _c_i, _c_i, _c_i, _c_i,
                                                       _c_p, _c_p, _c_p, _c_i, _c_p, _c_p,
                                                       _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_decode_layer_post_attn": (_c_i, [_c_p, _c_sz, _c_p, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p, _c_p,
                                            _c_p, _c_p, ctypes.c_float, _c_p, _c_p, _c_i,
                                            _c_p, _c_p, _c_p, _c_p, _c_p,
                                            _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                            _c_i, _c_i, _c_i, _c_i,
                                            _c_p, _c_p, _c_p, _c_i, _c_p, _c_p,
                                            _c_p, _c_sz, _c_p, _c_p, _c_p, _c_p, _c_i, ctypes.c_float, _c_i,
                                            _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_attn_decode_fused_partials": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, ctypes.c_float, _c_p, _c_p,
                                                _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p, _c_sz, _c_p]),
    "mxfp4_decode_stack_workspace_size": (_c_sz, [_c_i, _c_i, _c_i]),
    "mxfp4_decode_stack_reset": (_c_i, [_c_p, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_decode_stack_status": (_c_i, [_c_p, ctypes.POINTER(ctypes.c_int)]),
    "mxfp4_moe_decode_stack": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p,
                                      _c_i, _c_p, _c_sz, _c_p]),
    "mxfp4_embed_rows": (_c_i, [_c_p, _c_p, _c_i, _c_i, _c_p, _c_i, _c_p, _c_p]),
    "mxfp4_rmsnorm_quant": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "mxfp4_rmsnorm_lin_pq": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p, _c_p,
                                    _c_p, _c_i, _c_p, _c_p]),
    "mxfp4_qk_norm_rope_kv": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, ctypes.c_float, _c_p, _c_i, _c_i, _c_i, _c_i,
                                     _c_p, _c_p, _c_p, _c_i, _c_i, _c_p]),
    "mxfp4_argmax_workspace_size": (_c_sz, [_c_i, _c_i]),
    "mxfp4_argmax_advance": (_c_i, [_c_p, _c_i, _c_i, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_attn_decode_workspace_size": (_c_sz, [_c_i, _c_i, _c_i]),
    "mxfp4_attn_decode": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i,
                                 _c_p, _c_sz, _c_p]),
    "mxfp4_attn_decode_mx": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i,
                                    _c_p, _c_sz, _c_p]),
    "mxfp4_attn_decode_fused": (_c_i, [_c_p, _c_p, _c_p, ctypes.c_float, ctypes.c_float, _c_p, _c_p, _c_p, _c_p,
                                       _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p, _c_sz, _c_p]),
    "mxfp4_kv_write": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "mxfp4_moe_group": (_c_i, [_c_p, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p]),
    "mxfp4_route_topk": (_c_i, [_c_p, _c_i64, _c_i, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p]),
    "mxfp4_route_tables": (_c_i, [_c_p, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i,
                                  _c_p, _c_p, _c_p, _c_p, _c_p]),
    "mxfp4_moe_decode_batch_workspace_size": (_c_sz, [_c_i, _c_i, _c_i]),
    "mxfp4_moe_decode_batch": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i,
                                      _c_i, _c_i, _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_moe_decode_batch_noalloc": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i,
                                              _c_i, _c_i, _c_i, _c_i, _c_p, _c_p]),
    "mxfp4_moe_prefill_workspace_size": (_c_sz, [_c_i, _c_i, _c_i, _c_i, _c_i]),
    "mxfp4_moe_prefill": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                 _c_i, _c_i, _c_i, _c_i, _c_i, _c_p, _c_p, _c_sz, _c_p]),
    "mxfp4_moe_prefill_tab": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i,
                                     _c_p, _c_p, _c_sz, _c_p]),
}

# Optional exports added by later ABI versions are declared here as they land.
OPTIONAL_SIGNATURES = {}

_lib = None


class HipOpError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def load():
    """Load the HIP library (once).  Raises ImportError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"moe_fused_inference_amd: HIP library not built ({LIB_PATH}); "
            "run `python -m moe_fused_inference_amd.build` (or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in {**SIGNATURES, **OPTIONAL_SIGNATURES}.items():
        fn = getattr(lib, name, None)
        if fn is None:
            if name in OPTIONAL_SIGNATURES:
                continue
            raise ImportError(f"{LIB_PATH} does not export {name}")
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status, what):
    """Raise HipOpError with the library's message on a non-zero status."""
    if status != 0:
        msg = _lib.mxfp4_last_error().decode(errors="replace") if _lib is not None else ""
        raise HipOpError(f"{what} failed (status {status}): {msg}")


def ptr_array(ptrs):
    """Python ints -> ctypes array of void* (a host pointer table)."""
    arr = (ctypes.c_void_p * len(ptrs))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr
