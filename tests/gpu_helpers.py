"""Shared helpers of the GPU parity tests (imported by tests/test_gpu_*.py)."""
import numpy as np
import torch

from oracle import mxfp4 as fmt
from oracle import ops

DEV = "cuda"

# Per-op tolerance against the float64 oracle on the SAME quantized operands:
# products of E2M1 x E2M1 (or E4M3 x E2M1) with E8M0 scales are exact in fp32,
# so only the accumulation order differs.
COS_OP = 0.99999
REL_OP = 1e-4
# cos >= 0.999 and max-rel <= 1e-2,
# max-rel defined norm-wise as max|y - ref| / max|ref|.
COS_NS = 0.999
REL_NS = 1e-2


def log(msg):
    print(msg, flush=True)


def quantize_gpu(dext, w_bf16):
    """bf16 (n, k) cuda -> packed, scales (cuda u8) with the bit-exact HIP quantizer."""
    xq, xs = dext.prequant(w_bf16)
    return xq, xs


def rand_weight(dext, n, k, seed, std=0.02, device=DEV):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    w = (torch.randn((n, k), generator=g, device=device, dtype=torch.float32) * std).bfloat16()
    return quantize_gpu(dext, w)


def np_(t):
    return t.detach().cpu().numpy()


def assert_close(y, ref, cos_min=COS_OP, rel_max=REL_OP, what=""):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    c = ops.cos_sim(y, ref)
    r = ops.max_rel(y, ref)
    log(f"  {what}: cos={c:.9f} max_rel={r:.3e}")
    assert c >= cos_min, (what, c)
    assert r <= rel_max, (what, r)
    return c, r


def dequant(q, s, k=None):
    return fmt.dequant_rows(np_(q), np_(s), k)


def pool_layer(dext, n_exp, H, Mi, seed, chunk=16):
    """One MoE layer of n_exp experts with seeded bf16 N(0, 0.02) weights,
    quantized on the GPU by the bit-exact quantizer, stacked per projection as
    config 2 holds them: gate/up (n_exp, Mi, H/2) + (n_exp, Mi, H/32), down
    (n_exp, H, Mi/2) + (n_exp, H, Mi/32).  Experts are drawn `chunk` at a time."""
    from moe_fused_inference_amd import moe_layer
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    t = {}
    for nm, (n, k) in (("gate", (Mi, H)), ("up", (Mi, H)), ("down", (H, Mi))):
        wps, wss = [], []
        for e0 in range(0, n_exp, chunk):
            c = min(chunk, n_exp - e0)
            w = (torch.randn((c * n, k), generator=g, device=DEV) * 0.02).bfloat16()
            q, s = dext.prequant(w)
            wps.append(q.view(c, n, k // 2))
            wss.append(s.view(c, n, k // 32))
        t[nm + "_wp"] = torch.cat(wps).contiguous()
        t[nm + "_ws"] = torch.cat(wss).contiguous()
    return moe_layer.StackedExperts(**t)
