"""Packed MXFP4 checkpoint mirror -> expert weights resident in HBM.

Reads the mirror the reference's quantizer writes
(quant/quantize_mxfp4.py:41-87 ShardWriter, :175-223 run_quantization):

    manifest.json                    {"format": "mxfp4-1x32-e8m0-e2m1", "block_size": 32,
                                      "tensors": {source name: {"orig_shape": [n, k],
                                      "padded_k": kp, "data_key", "scale_key", ...}}}
    model.safetensors                (one shard), or
    model-0000i-of-0000n.safetensors + model.safetensors.index.json {"weight_map": {key: shard}}

where each expert projection `model.layers.L.mlp.experts.e.{gate,up,down}_proj.weight`
is stored as `<name>.fp4_data` (the n*kp/2 packed E2M1 bytes, row-major,
low nibble first) and `<name>.fp4_scale` (uint8 E8M0 codes (n, kp/32)).

Two consumers:
  * ``expert_specs(L)`` -- the reference's per-expert spec dicts
    {"gate"/"up"/"down": {"wp", "wsc", "K"}} on the device, as
    runtime/weight_store.py:270-289 (variant "mxfp4_mma") returns them, for
    the drop-in operators;
  * ``stacked_layer(L)`` -- the layer's experts stacked back to back
    (moe_layer.StackedExperts), the layout of the fused decode layer and the
    grouped prefill MoE; the bytes of every expert slice are identical to the
    shard's.

Tensors are read through safetensors' memory-mapped numpy views (nothing is
unpickled) and copied to the device one layer at a time through a reusable
pinned staging buffer.
"""
import json
import os
import re

import numpy as np

FORMAT = "mxfp4-1x32-e8m0-e2m1"
BLOCK = 32
PROJS = ("gate", "up", "down")
_EXPERT_RE = re.compile(r"^model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate|up|down)_proj\.weight$")


class MirrorError(RuntimeError):
    """The mirror is missing, malformed or inconsistent."""


class Mxfp4Mirror:
    """Read-only view of one MXFP4 mirror directory."""

    def __init__(self, mirror_dir):
        from safetensors import safe_open

        self.dir = mirror_dir
        mpath = os.path.join(mirror_dir, "manifest.json")
        if not os.path.exists(mpath):
            raise MirrorError(f"{mirror_dir}: no manifest.json")
        with open(mpath) as f:
            self.manifest = json.load(f)
        if self.manifest.get("format") != FORMAT or int(self.manifest.get("block_size", 0)) != BLOCK:
            raise MirrorError(f"{mirror_dir}: format {self.manifest.get('format')!r} / block "
                              f"{self.manifest.get('block_size')!r}, expected {FORMAT!r} / {BLOCK}")
        self.info = self.manifest.get("tensors", {})
        ipath = os.path.join(mirror_dir, "model.safetensors.index.json")
        if os.path.exists(ipath):
            with open(ipath) as f:
                self.index = json.load(f)["weight_map"]
            shards = sorted(set(self.index.values()))
        else:
            self.index = None
            shards = sorted(f for f in os.listdir(mirror_dir) if f.endswith(".safetensors"))
        if not shards:
            raise MirrorError(f"{mirror_dir}: no safetensors shards")
        self.handles = {s: safe_open(os.path.join(mirror_dir, s), framework="numpy") for s in shards}
        self.experts = {}   # layer -> {expert id -> {proj: source name}}
        for name in self.info:
            m = _EXPERT_RE.match(name)
            if m:
                L, e, p = int(m.group(1)), int(m.group(2)), m.group(3)
                self.experts.setdefault(L, {}).setdefault(e, {})[p] = name

    # ------------------------------------------------------------------ raw access
    def _get(self, key):
        if self.index is not None:
            shard = self.index.get(key)
            if shard is None:
                raise MirrorError(f"{key} is not in the shard index")
            return self.handles[shard].get_tensor(key)
        for h in self.handles.values():
            if key in h.keys():
                return h.get_tensor(key)
        raise MirrorError(f"{key} is in no shard")

    def packed(self, name):
        """Source tensor name -> (wp (n, kp/2) u8, wsc (n, kp/32) u8, K) as numpy."""
        info = self.info.get(name)
        if info is None:
            raise MirrorError(f"{name} is not in the manifest")
        n, k = (int(v) for v in info["orig_shape"])
        kp = int(info["padded_k"])
        if kp % BLOCK or kp < k:
            raise MirrorError(f"{name}: padded_k={kp} for K={k}")
        data = self._get(info["data_key"])
        scale = self._get(info["scale_key"])
        if data.dtype != np.uint8 or data.size != n * kp // 2:
            raise MirrorError(f"{name}: data has {data.size} {data.dtype} entries, expected {n * kp // 2} uint8")
        if scale.dtype != np.uint8 or scale.size != n * kp // BLOCK:
            raise MirrorError(f"{name}: scales have {scale.size} {scale.dtype} entries, expected {n * kp // BLOCK}")
        return data.reshape(n, kp // 2), scale.reshape(n, kp // BLOCK), k

    def layers(self):
        """Layer indices that have expert tensors."""
        return sorted(self.experts)

    def expert_ids(self, L):
        return sorted(self.experts.get(L, {}))

    # ------------------------------------------------------------------ consumers
    def expert_specs(self, L, device="cuda", ids=None):
        """{e: {"gate"/"up"/"down": {"wp", "wsc", "K"}}} on `device` --
        runtime/weight_store.py:270-289 (variant "mxfp4_mma")."""
        import torch

        out = {}
        for e in (self.expert_ids(L) if ids is None else ids):
            names = self.experts.get(L, {}).get(int(e))
            if names is None or set(names) != set(PROJS):
                raise MirrorError(f"layer {L} expert {e}: missing projections")
            spec = {}
            for p in PROJS:
                wp, ws, k = self.packed(names[p])
                spec[p] = {"wp": torch.from_numpy(np.ascontiguousarray(wp)).to(device),
                           "wsc": torch.from_numpy(np.ascontiguousarray(ws)).to(device), "K": k}
            out[int(e)] = spec
        return out

    def stacked_shapes(self, L):
        """(n_experts, H, Mi) of layer L after checking that experts 0..n-1
        are all present with gate/up (Mi, H) and down (H, Mi), H and Mi
        multiples of 32."""
        ids = self.expert_ids(L)
        if not ids or ids != list(range(len(ids))):
            raise MirrorError(f"layer {L}: experts {ids[:4]}... are not 0..n-1")
        shapes = {}
        for e in ids:
            names = self.experts[L][e]
            if set(names) != set(PROJS):
                raise MirrorError(f"layer {L} expert {e}: missing projections")
            for p in PROJS:
                shapes.setdefault(p, set()).add(tuple(int(v) for v in self.info[names[p]]["orig_shape"]))
        if any(len(v) != 1 for v in shapes.values()):
            raise MirrorError(f"layer {L}: experts differ in shape {shapes}")
        (mi, h), = shapes["gate"]
        if shapes["up"] != {(mi, h)} or shapes["down"] != {(h, mi)} or h % BLOCK or mi % BLOCK:
            raise MirrorError(f"layer {L}: shapes {shapes} are not gate/up (Mi, H), down (H, Mi) with 32 | H, Mi")
        return len(ids), h, mi

    def stacked_arrays(self, L):
        """Layer L as six host arrays {gate_wp: (n, Mi, H/2), gate_ws: (n, Mi, H/32), up_*, down_wp:
        (n, H, Mi/2), down_ws: (n, H, Mi/32)} (uint8)."""
        n, h, mi = self.stacked_shapes(L)
        out = {}
        for p, (rows, cols) in zip(PROJS, ((mi, h), (mi, h), (h, mi))):
            wp = np.empty((n, rows, cols // 2), np.uint8)
            ws = np.empty((n, rows, cols // BLOCK), np.uint8)
            for e in range(n):
                wp[e], ws[e], _ = self.packed(self.experts[L][e][p])
            out[p + "_wp"], out[p + "_ws"] = wp, ws
        return out

    def stacked_layer(self, L, device="cuda", staging=None):
        """Layer L's experts stacked back to back on `device`
        (moe_layer.StackedExperts).  `staging`: an optional dict reused across
        calls for the pinned host buffers."""
        import torch

        from .moe_layer import StackedExperts

        n, h, mi = self.stacked_shapes(L)
        staging = {} if staging is None else staging
        dev = {}
        for p, (rows, cols) in zip(PROJS, ((mi, h), (mi, h), (h, mi))):
            for kind, width in (("_wp", cols // 2), ("_ws", cols // BLOCK)):
                shape = (n, rows, width)
                buf = staging.get(p + kind)
                if buf is None or tuple(buf.shape) != shape:
                    buf = torch.empty(shape, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
                    staging[p + kind] = buf
                host = buf.numpy()
                for e in range(n):
                    wp, ws, _ = self.packed(self.experts[L][e][p])
                    host[e] = wp if kind == "_wp" else ws
                t = torch.empty(shape, dtype=torch.uint8, device=device)
                t.copy_(buf, non_blocking=True)
                dev[p + kind] = t
        if torch.cuda.is_available():
            torch.cuda.current_stream().synchronize()   # the staging buffers are reused by the next call
        return StackedExperts(**dev)
