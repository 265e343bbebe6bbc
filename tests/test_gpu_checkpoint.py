"""End to end from checkpoint files: a mirror in the reference's format
(tests/mirror_writer.py) loaded by moe_fused_inference_amd.checkpoint into
HBM drives the fused decode layer and the drop-in ops; results against the
oracle on the mirror's own bytes."""
import numpy as np
import pytest
import torch

from moe_fused_inference_amd import checkpoint as ck
from moe_fused_inference_amd import moe_layer
from oracle import ops
from tests import mirror_writer as mw
from tests.gpu_helpers import COS_NS, DEV, REL_NS, assert_close, np_

pytestmark = pytest.mark.gpu


def test_fused_layer_from_mirror(dext, tmp_path):
    n_exp, H, Mi, E = 8, 1024, 256, 4
    w = mw.random_layers(2, n_exp, H, Mi, seed=11)
    packed = mw.write_mirror(str(tmp_path), w, max_shard_bytes=3 << 20)
    m = ck.Mxfp4Mirror(str(tmp_path))
    staging = {}
    stacks = [m.stacked_layer(L, DEV, staging) for L in (0, 1)]
    for L, st in enumerate(stacks):
        assert np.array_equal(np_(st.down_wp[5]), packed[mw.expert_name(L, 5, "down")][0])
    g = torch.Generator(device=DEV)
    g.manual_seed(3)
    x = torch.randn((1, H), generator=g, device=DEV).bfloat16()
    ids, wts = [6, 1, 3, 0], [0.4, 0.3, 0.2, 0.1]
    out, _ = moe_layer.decode_layer(x, ids, wts, stacks[1], ws=moe_layer.workspace(E, Mi, H))
    torch.cuda.synchronize()
    experts = {e: tuple(packed[mw.expert_name(1, e, p)] for p in ("gate", "up", "down")) for e in ids}
    ref = ops.decode_layer_ref(np_(x.float()), np.array([ids]), np.array([wts]), experts)[0]
    assert_close(np_(out), ref, COS_NS, REL_NS, what="fused layer from the mirror")
    # the drop-in ops on the reference's spec dicts from the same mirror give
    # the same bits as on the stacked layer's slices
    specs = m.expert_specs(1, device=DEV, ids=ids)
    xq, xs = dext.prequant(x)

    def dropin(get):
        gu = dext.moe_gateup(xq, xs, [get(e, "gate", "wp") for e in ids] + [get(e, "up", "wp") for e in ids],
                             [get(e, "gate", "ws") for e in ids] + [get(e, "up", "ws") for e in ids], E, 1, Mi, H)
        yd = dext.moe_down(gu, [get(e, "down", "wp") for e in ids], [get(e, "down", "ws") for e in ids], E, 1, H, Mi)
        return dext.moe_combine(yd, torch.tensor([wts], dtype=torch.float32, device=DEV), 1)[0]

    a = dropin(lambda e, p, k: specs[e][p]["wp" if k == "wp" else "wsc"])
    b = dropin(lambda e, p, k: getattr(stacks[1], f"{p}_{k}")[e])
    torch.cuda.synchronize()
    assert torch.equal(a, b)
