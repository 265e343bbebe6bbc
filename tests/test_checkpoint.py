"""The packed-checkpoint loader (moe_fused_inference_amd.checkpoint) on
mirrors written in the reference's format (tests/mirror_writer.py): every
stacked expert slice must hold exactly the shard's bytes."""
import json
import os

import numpy as np
import pytest
import torch

from moe_fused_inference_amd import checkpoint as ck
from tests import mirror_writer as mw


def _check_layer(m, packed, L, n_exp):
    arr = m.stacked_arrays(L)
    for e in range(n_exp):
        for p in ("gate", "up", "down"):
            q, s = packed[mw.expert_name(L, e, p)]
            assert np.array_equal(arr[p + "_wp"][e], q) and np.array_equal(arr[p + "_ws"][e], s)


@pytest.mark.parametrize("shard_bytes", [1 << 40, 4000])
def test_mirror_round_trip(tmp_path, shard_bytes):
    n_layers, n_exp, H, Mi = 2, 3, 64, 32
    w = mw.random_layers(n_layers, n_exp, H, Mi, seed=1)
    packed = mw.write_mirror(str(tmp_path), w, max_shard_bytes=shard_bytes,
                             extra={"model.norm.weight": np.ones(H)})
    sharded = os.path.exists(tmp_path / "model.safetensors.index.json")
    assert sharded == (shard_bytes < 1 << 40)
    m = ck.Mxfp4Mirror(str(tmp_path))
    assert m.layers() == [0, 1] and m.expert_ids(1) == [0, 1, 2]
    assert m.stacked_shapes(0) == (n_exp, H, Mi)
    for L in range(n_layers):
        _check_layer(m, packed, L, n_exp)
    specs = m.expert_specs(1, device="cpu", ids=[2])
    q, s = packed[mw.expert_name(1, 2, "down")]
    assert specs[2]["down"]["K"] == Mi
    assert np.array_equal(specs[2]["down"]["wp"].numpy(), q) and np.array_equal(specs[2]["down"]["wsc"].numpy(), s)
    assert specs[2]["gate"]["wp"].dtype == torch.uint8 and tuple(specs[2]["gate"]["wp"].shape) == (Mi, H // 2)


def test_padded_k_is_read_with_its_padding(tmp_path):
    rng = np.random.default_rng(2)
    w = {mw.expert_name(0, 0, "gate"): rng.standard_normal((8, 40)).astype(np.float32)}
    packed = mw.write_mirror(str(tmp_path), w)
    m = ck.Mxfp4Mirror(str(tmp_path))
    wp, ws, k = m.packed(mw.expert_name(0, 0, "gate"))
    assert k == 40 and wp.shape == (8, 32) and ws.shape == (8, 2)
    assert np.array_equal(wp, packed[mw.expert_name(0, 0, "gate")][0])
    with pytest.raises(ck.MirrorError, match="missing projections"):
        m.stacked_shapes(0)


def test_malformed_mirrors_are_rejected(tmp_path):
    w = mw.random_layers(1, 2, 64, 32, seed=3)
    bad = tmp_path / "fmt"
    mw.write_mirror(str(bad), w, fmt_name="mxfp8")
    with pytest.raises(ck.MirrorError, match="format"):
        ck.Mxfp4Mirror(str(bad))
    gap = tmp_path / "gap"
    del w[mw.expert_name(0, 0, "gate")], w[mw.expert_name(0, 0, "up")], w[mw.expert_name(0, 0, "down")]
    mw.write_mirror(str(gap), w)
    with pytest.raises(ck.MirrorError, match="not 0..n-1"):
        ck.Mxfp4Mirror(str(gap)).stacked_shapes(0)
    odd = tmp_path / "odd"
    w2 = mw.random_layers(1, 2, 64, 32, seed=4)
    w2[mw.expert_name(0, 1, "up")] = np.zeros((32, 96), np.float32)
    mw.write_mirror(str(odd), w2)
    with pytest.raises(ck.MirrorError, match="differ in shape"):
        ck.Mxfp4Mirror(str(odd)).stacked_shapes(0)
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(ck.MirrorError, match="no manifest"):
        ck.Mxfp4Mirror(str(empty))
    # a manifest entry whose data tensor has the wrong size
    trunc = tmp_path / "trunc"
    mw.write_mirror(str(trunc), mw.random_layers(1, 1, 64, 32, seed=5))
    man = json.load(open(trunc / "manifest.json"))
    man["tensors"][mw.expert_name(0, 0, "gate")]["orig_shape"] = [33, 64]
    json.dump(man, open(trunc / "manifest.json", "w"))
    with pytest.raises(ck.MirrorError, match="data has"):
        ck.Mxfp4Mirror(str(trunc)).packed(mw.expert_name(0, 0, "gate"))
