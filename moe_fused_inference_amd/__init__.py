"""MI355X (gfx950) MXFP4 MoE hot path: a from-scratch HIP implementation of the
decode grouped-expert ops, the block-scaled MXFP4 GEMM and the activation
quantizer of shuimenwang/moe_fused_inference, behind the reference's own
operator surface (``fp4_ext.get_ext()`` / ``fp4_ext.get_decode_ext()``).

The compute runs in ``lib/libmxfp4_hip.so`` (C ABI: include/mxfp4_hip.h);
this package holds only the host-side mirror of the reference interface.
"""
from .fp4_ext import get_decode_ext, get_ext  # noqa: F401

__all__ = ["get_ext", "get_decode_ext"]
