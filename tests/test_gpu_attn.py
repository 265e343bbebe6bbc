"""GPU parity of decode attention over the FP8 KV cache and of the KV write
(mxfp4_attn_decode, mxfp4_kv_write), the reference's attn_decode / kv_write
(src/ext/mxfp4_decode.cu:352-490).

Oracle: oracle/attn.py, pinned in tests/test_oracle_attn.py.  The KV bytes
are compared bit-exactly; attention output against the float64 oracle on the
same cache bytes with the per-op tolerance (cos >= 0.99999, norm-wise
max-rel <= 1e-4), the raw scores written to `sc` with max-rel <= 1e-5.
"""
import ctypes

import numpy as np
import pytest
import torch

from moe_fused_inference_amd import _lib
from oracle import attn
from oracle import mxfp4 as fmt
from tests.gpu_helpers import DEV, assert_close, log, np_

pytestmark = pytest.mark.gpu


def _bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).bfloat16()


def _mixed_values(rng, shape):
    """bf16 values over the codec's regimes: sub-2^-6, normal, ties, >= 248."""
    x = rng.standard_normal(shape).astype(np.float32)
    scale = rng.choice(np.array([1e-3, 0.02, 0.5, 3.0, 60.0, 400.0], np.float32), size=shape)
    x *= scale
    flat = x.reshape(-1)
    ties = np.array([1.0625, -1.1875, 0.03125 * 1.0625, 17.0, 240.0, 248.0, -250.0, 2.0 ** -7, 0.0, -0.0],
                    np.float32)
    flat[:ties.size] = ties
    return _bf16(x)


@pytest.mark.parametrize("M,Hkv,base,max_pos", [(1, 4, 5, 64), (9, 4, 30, 64), (4, 8, 62, 64), (3, 2, -1, 16)])
def test_kv_write_bit_exact(dext, M, Hkv, base, max_pos):
    rng = np.random.default_rng(M * 100 + Hkv + max_pos)
    D = 128
    k, v = _mixed_values(rng, (M, Hkv, D)), _mixed_values(rng, (M, Hkv, D))
    init_k = rng.integers(0, 256, size=(max_pos, Hkv, D), dtype=np.uint8)
    init_v = rng.integers(0, 256, size=(max_pos, Hkv, D), dtype=np.uint8)
    kvk, kvv = torch.from_numpy(init_k.copy()).to(DEV), torch.from_numpy(init_v.copy()).to(DEV)
    dpos = torch.tensor([base], dtype=torch.int32, device=DEV)
    dext.kv_write(k.to(DEV), v.to(DEV), kvk, kvv, dpos, M)
    torch.cuda.synchronize()
    wk, wv = attn.kv_write_ref(k.float().numpy(), v.float().numpy(), init_k.copy(), init_v.copy(), base)
    assert np.array_equal(np_(kvk), wk) and np.array_equal(np_(kvv), wv)
    written = max(0, min(M, max_pos - base)) if base >= 0 else 0
    log(f"  kv_write M={M} Hkv={Hkv} base={base}: {written} rows written, bit-exact")


def _cache(rng, max_pos, Hkv, D, scale=0.5):
    return attn.e4m3_ref_encode(rng.standard_normal((max_pos, Hkv, D)).astype(np.float32) * scale)


@pytest.mark.parametrize("M,Hq,Hkv,max_pos,base", [(1, 32, 4, 4096, 4095), (1, 32, 4, 4096, 0),
                                                  (9, 32, 4, 4096, 2000), (2, 8, 8, 256, 100),
                                                  (3, 16, 1, 300, 250), (1, 4, 2, 128, 70),
                                                  # more than 64 chunks: the two-pass merge
                                                  (2, 32, 4, 8192, 6000), (1, 8, 2, 8192, 8191)])
def test_attn_decode_vs_oracle(dext, M, Hq, Hkv, max_pos, base):
    rng = np.random.default_rng(Hq * 7 + max_pos + base)
    D = 128
    kvk_np, kvv_np = _cache(rng, max_pos, Hkv, D), _cache(rng, max_pos, Hkv, D)
    q = _bf16(rng.standard_normal((M, Hq, D)))
    sc = torch.full((M, Hq, max_pos), float("nan"), dtype=torch.float32, device=DEV)
    o = dext.attn_decode(q.to(DEV), torch.from_numpy(kvk_np).to(DEV), torch.from_numpy(kvv_np).to(DEV),
                         torch.tensor([base], dtype=torch.int32, device=DEV), sc, M)
    torch.cuda.synchronize()
    ref, scores = attn.attn_decode_ref(q.float().numpy(), kvk_np, kvv_np, base)
    assert_close(np_(o), ref, what=f"attn_decode M={M} Hq={Hq} Hkv={Hkv} S={base + 1}..")
    for m in range(M):
        S = base + m + 1
        got = np_(sc[m, :, :S]).astype(np.float64)
        err = np.abs(got - scores[m]).max() / np.abs(scores[m]).max()
        assert err <= 1e-5, (m, err)


def test_attn_decode_rows_past_the_cache_are_skipped(dext):
    """Token rows whose position falls outside [0, max_pos) write nothing
    (src/ext/mxfp4_decode.cu:378,410)."""
    rng = np.random.default_rng(5)
    M, Hq, Hkv, D, max_pos = 3, 8, 2, 128, 64
    kvk = torch.from_numpy(_cache(rng, max_pos, Hkv, D)).to(DEV)
    kvv = torch.from_numpy(_cache(rng, max_pos, Hkv, D)).to(DEV)
    q = _bf16(rng.standard_normal((M, Hq, D))).to(DEV)
    o = torch.full((M, Hq, D), float("nan"), dtype=torch.float32, device=DEV)
    sc = torch.zeros((M, Hq, max_pos), dtype=torch.float32, device=DEV)
    dpos = torch.tensor([max_pos - 1], dtype=torch.int32, device=DEV)
    lib = _lib.load()
    wsb = lib.mxfp4_attn_decode_workspace_size(M, Hq, max_pos)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    _lib.check(lib.mxfp4_attn_decode(q.data_ptr(), kvk.data_ptr(), kvv.data_ptr(), dpos.data_ptr(), sc.data_ptr(),
                                     o.data_ptr(), M, Hq, Hkv, D, max_pos, ws.data_ptr(), wsb,
                                     torch.cuda.current_stream().cuda_stream), "attn_decode")
    torch.cuda.synchronize()
    assert not torch.isnan(o[0]).any() and torch.isnan(o[1:]).all()
    ref, _ = attn.attn_decode_ref(q.float().cpu().numpy(), np_(kvk), np_(kvv), max_pos - 1)
    assert_close(np_(o[0]), ref[0], what="last cache row")


def test_attn_decode_in_graph_follows_dpos(dext):
    """attn_decode + kv_write captured once; dpos updated between replays
    (how runtime/model_runner_v3.py:98-126 drives them)."""
    rng = np.random.default_rng(6)
    M, Hq, Hkv, D, max_pos = 1, 32, 4, 128, 512
    kvk_np, kvv_np = _cache(rng, max_pos, Hkv, D), _cache(rng, max_pos, Hkv, D)
    kvk, kvv = torch.from_numpy(kvk_np.copy()).to(DEV), torch.from_numpy(kvv_np.copy()).to(DEV)
    q = _bf16(rng.standard_normal((M, Hq, D))).to(DEV)
    k = _bf16(rng.standard_normal((M, Hkv, D))).to(DEV)
    v = _bf16(rng.standard_normal((M, Hkv, D))).to(DEV)
    dpos = torch.tensor([10], dtype=torch.int32, device=DEV)
    sc = torch.empty((M, Hq, max_pos), dtype=torch.float32, device=DEV)
    out = torch.empty((M, Hq, D), dtype=torch.float32, device=DEV)

    def step():
        dext.kv_write(k, v, kvk, kvv, dpos, M)
        out.copy_(dext.attn_decode(q, kvk, kvv, dpos, sc, M))

    step()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            step()
    torch.cuda.synchronize()
    ck, cv = kvk_np.copy(), kvv_np.copy()
    attn.kv_write_ref(k.float().cpu().numpy(), v.float().cpu().numpy(), ck, cv, 10)
    for pos in (50, 300, 511):
        dpos.fill_(pos)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        attn.kv_write_ref(k.float().cpu().numpy(), v.float().cpu().numpy(), ck, cv, pos)
        assert np.array_equal(np_(kvk), ck) and np.array_equal(np_(kvv), cv)
        ref, _ = attn.attn_decode_ref(q.float().cpu().numpy(), ck, cv, pos)
        assert_close(np_(out), ref, what=f"graph replay at dpos={pos}")


@pytest.mark.parametrize("M,Hq,Hkv,max_pos,base", [(1, 32, 4, 4096, 4095), (4, 32, 4, 1000, 700), (3, 16, 1, 200, 0),
                                                   (2, 8, 8, 128, 63)])
def test_attn_decode_mx_quantized_output(M, Hq, Hkv, max_pos, base):
    """The attention output written as MXFP4 rows of bf16(o) equals
    mxfp4_quantize_rows (bf16 mode) of the fp32 output bit for bit, o itself
    equals the plain entry point's bit for bit, on three calls in a row
    that share one workspace."""
    lib = _lib.load()
    rng = np.random.default_rng(M * 1000 + base)
    D = 128
    kvk = torch.from_numpy(_cache(rng, max_pos, Hkv, D)).to(DEV)
    kvv = torch.from_numpy(_cache(rng, max_pos, Hkv, D)).to(DEV)
    dpos = torch.tensor([base], dtype=torch.int32, device=DEV)
    sc = torch.zeros((M, Hq, max_pos), dtype=torch.float32, device=DEV)
    wsb = lib.mxfp4_attn_decode_workspace_size(M, Hq, max_pos)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    for call in range(3):
        q = _bf16(rng.standard_normal((M, Hq, D)) * (1 + call)).to(DEV)
        o1 = torch.zeros((M, Hq, D), dtype=torch.float32, device=DEV)
        o2 = torch.zeros((M, Hq, D), dtype=torch.float32, device=DEV)
        oq = torch.zeros((M, Hq * D // 2), dtype=torch.uint8, device=DEV)
        os_ = torch.zeros((M, Hq * D // 32), dtype=torch.uint8, device=DEV)
        _lib.check(lib.mxfp4_attn_decode(q.data_ptr(), kvk.data_ptr(), kvv.data_ptr(), dpos.data_ptr(), sc.data_ptr(),
                                         o1.data_ptr(), M, Hq, Hkv, D, max_pos, ws.data_ptr(), wsb, st), "attn_decode")
        _lib.check(lib.mxfp4_attn_decode_mx(q.data_ptr(), kvk.data_ptr(), kvv.data_ptr(), dpos.data_ptr(),
                                            sc.data_ptr(), o2.data_ptr(), oq.data_ptr(), os_.data_ptr(), M, Hq, Hkv, D,
                                            max_pos, ws.data_ptr(), wsb, st), "attn_decode_mx")
        torch.cuda.synchronize()
        live = [m for m in range(M) if base + m < max_pos]
        assert torch.equal(o1[live], o2[live]), f"call {call}"
        rq, rs = fmt.quantize_rows(fmt.bf16_round(np_(o2).reshape(M, Hq * D)))
        assert np.array_equal(np_(oq)[live], rq[live]) and np.array_equal(np_(os_)[live], rs[live]), f"call {call}"
        ref, _ = attn.attn_decode_ref(q.float().cpu().numpy(), np_(kvk), np_(kvv), base)
        assert_close(np_(o2)[live], ref[live], what=f"attn_decode_mx call {call}")
