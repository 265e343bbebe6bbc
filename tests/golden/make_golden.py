"""Writes the golden fixtures under tests/golden/.

mxfp4_kat.json   the known-answer tests of the reference's format self-test
                 (quant/fp4_format.py:154-198), written out as data:
                 inputs and expected outputs only.
quant_vectors.npz seeded activation/weight rows and their MXFP4 encoding by
                 the CPU oracle, for the shapes the reference's prequant test
                 uses (tests/correctness/test_mxfp4_decode.py:57) plus edge
                 rows (zero block, tiny negatives, exact ties, odd K).  These
                 are regression vectors of the oracle, which is itself pinned
                 by the KATs and the exhaustive sweeps in tests/test_oracle_format.py.

Run from the repo root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import mxfp4 as fmt  # noqa: E402


def kat():
    return {
        "source": "quant/fp4_format.py:154-198 (reference self-test), restated as data",
        # 1) every code decodes; code 8 (-0.0) re-quantizes to 0 (:157-163)
        "decode_all": {"codes": list(range(16)),
                       "values": [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                                  -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]},
        "requantize_all": {"codes": list(range(16)),
                           "expected": [0, 1, 2, 3, 4, 5, 6, 7, 0, 9, 10, 11, 12, 13, 14, 15]},
        # 2) known points (:166-171)
        "encode_points": [[1.7, 1.5], [1.5, 1.5], [0.25, 0.5], [7.0, 6.0], [-3.0, -3.0]],
        "decode_points": [[15, -6.0], [1, 0.5]],
        # 3) E8M0 block scale (:174-178): amax -> scale
        "scale_points": [[5.0, 1.0], [6.0, 1.0], [6.1, 2.0], [12.0, 2.0], [0.5, 0.125]],
        # 5) LSB-first packing with odd pad (:187-191)
        "pack": {"codes": [0, 7, 15, 1, 3], "bytes": [0x70, 0x1F, 0x03], "pad": 1},
        # 6) 64-element linspace chain (:194-198): quantize/pack/unpack round trip
        "linspace": {"start": -6.0, "stop": 6.0, "num": 64},
    }


def edge_rows():
    rows = []
    # all-zero block then a block of exact midpoints (ties go up) at scale 1
    r = np.zeros(64, np.float32)
    r[32:39] = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    r[39] = 6.0                       # amax 6 -> scale 1
    r[40:47] = [-0.25, -0.75, -1.25, -1.75, -2.5, -3.5, -5.0]
    rows.append(r)
    # tiny negatives next to a large value: magnitude 0 with sign -> code 8
    r = np.zeros(64, np.float32)
    r[0] = 96.0
    r[1:8] = -np.float32(2.0 ** -20)
    r[33] = np.float32(3.0) * np.float32(2.0 ** -126)   # denormal-range amax block
    r[34] = -np.float32(2.0 ** -133)                    # smallest bf16 denormal
    r[40] = np.float32(np.inf)                          # inf amax -> scale code 127
    r[41] = np.float32(-7.5)
    rows.append(r)
    out = np.stack(rows)
    assert np.array_equal(fmt.bf16_round(out), out), "edge rows must be bf16-exact"
    return out


def vectors():
    out = {}
    rng = np.random.default_rng(0)
    for M, K in [(1, 64), (1, 2048), (3, 768), (2, 100), (2, 33)]:
        x = rng.standard_normal((M, K)).astype(np.float32) * 0.5
        x[rng.random((M, K)) < 0.01] *= 4.0
        x = fmt.bf16_round(x)
        q, s = fmt.quantize_rows(x)
        out[f"x_{M}x{K}"] = x
        out[f"q_{M}x{K}"] = q
        out[f"s_{M}x{K}"] = s
    e = edge_rows()
    q, s = fmt.quantize_rows(e)
    out["x_edge"], out["q_edge"], out["s_edge"] = e, q, s
    return out


if __name__ == "__main__":
    with open(os.path.join(HERE, "mxfp4_kat.json"), "w") as f:
        json.dump(kat(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "quant_vectors.npz"), **vectors())
    print("wrote", os.listdir(HERE))
