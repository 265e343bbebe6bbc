"""Writes small MXFP4 checkpoint mirrors in the reference's on-disk format
(quant/quantize_mxfp4.py:41-87 ShardWriter, :175-223 run_quantization) for
the loader tests: the expert tensors quantized by the oracle quantizer
(bit-exact to quant/quantize_mxfp4.py:110-160), stored as `<name>.fp4_data`
(flat packed bytes) and `<name>.fp4_scale` (E8M0 codes), a manifest, and one
shard or several shards plus model.safetensors.index.json.  Test
infrastructure."""
import json
import os

import numpy as np
from safetensors.numpy import save_file

from oracle import mxfp4 as fmt


def expert_name(L, e, p):
    return f"model.layers.{L}.mlp.experts.{e}.{p}_proj.weight"


def write_mirror(out_dir, weights, max_shard_bytes=1 << 40, extra=None, fmt_name="mxfp4-1x32-e8m0-e2m1"):
    """weights: {source name: fp32 (n, k)}; extra: {name: array} copied
    as-is.  Returns {source name: (packed (n, kp/2), scales (n, kp/32))}."""
    os.makedirs(out_dir, exist_ok=True)
    buf, nbytes, tmp, weight_map = {}, 0, [], {}

    def flush():
        nonlocal buf, nbytes
        if buf:
            fn = f"tmp-{len(tmp) + 1:05d}.safetensors"
            save_file(buf, os.path.join(out_dir, fn))
            for k in buf:
                weight_map[k] = fn
            tmp.append(fn)
            buf, nbytes = {}, 0

    def add(k, a):
        nonlocal nbytes
        buf[k] = np.ascontiguousarray(a)
        nbytes += a.nbytes
        if nbytes >= max_shard_bytes:
            flush()

    manifest = {"format": fmt_name, "block_size": 32, "scale_type": "e8m0_power_of_2", "tensors": {}}
    packed = {}
    for name, w in weights.items():
        q, s = fmt.quantize_rows(w)
        n, k = w.shape
        kp = s.shape[1] * 32
        dk, sk = name + ".fp4_data", name + ".fp4_scale"
        add(dk, q.reshape(-1))
        add(sk, s)
        manifest["tensors"][name] = {"orig_shape": [n, k], "orig_dtype": "torch.bfloat16", "padded_k": kp,
                                     "pad": kp - k, "n_elements": n * k, "scale_shape": list(s.shape),
                                     "scale_dtype": "e8m0_uint8", "data_key": dk, "scale_key": sk,
                                     "fp8_scale_inv_present": False}
        packed[name] = (q, s)
    for name, a in (extra or {}).items():
        add(name, np.asarray(a, np.float32))
    flush()
    if len(tmp) == 1:
        os.replace(os.path.join(out_dir, tmp[0]), os.path.join(out_dir, "model.safetensors"))
    else:
        final = {}
        for i, t in enumerate(tmp, 1):
            f = f"model-{i:05d}-of-{len(tmp):05d}.safetensors"
            os.replace(os.path.join(out_dir, t), os.path.join(out_dir, f))
            final[t] = f
        with open(os.path.join(out_dir, "model.safetensors.index.json"), "w") as fh:
            json.dump({"metadata": {"total_size": 0}, "weight_map": {k: final[v] for k, v in weight_map.items()}}, fh)
    with open(os.path.join(out_dir, "manifest.json"), "w") as fh:
        json.dump(manifest, fh)
    return packed


def random_layers(n_layers, n_exp, H, Mi, seed):
    rng = np.random.default_rng(seed)
    w = {}
    for L in range(n_layers):
        for e in range(n_exp):
            for p, shp in (("gate", (Mi, H)), ("up", (Mi, H)), ("down", (H, Mi))):
                w[expert_name(L, e, p)] = (rng.standard_normal(shp) * 0.02).astype(np.float32)
    return w
