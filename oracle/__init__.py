"""CPU oracle for the MXFP4 MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's MXFP4
path so that the HIP kernels can be checked against it.  It is a checker,
never the thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``moe_fused_inference_amd``) never imports this package and fails loudly when
its HIP library is missing.

Modules
-------
``mxfp4``  the format: E2M1 codec, E8M0 block scale, LSB-first nibble packing,
           the row quantizer and dequantizer (reference ``quant/fp4_format.py``,
           ``quant/quantize_mxfp4.py``, ``runtime/weight_store.py``).
``ops``    per-operator references (prequant, forward, lin_pq, moe_gateup,
           moe_down, moe_combine), routing, the token->expert grouping, the
           fused decode-layer reference and the dequant+BF16 CPU baseline.
``mxfp4_oracle.c``  an independent C restatement of the quantizer, used by the
           tests for exhaustive sweeps and as a second implementation that the
           numpy one is cross-checked against.

Parity pinning (what checks each function; see tests/test_oracle_*.py):
  E2M1 encode/decode   reference KATs (quant/fp4_format.py:157-171) + exhaustive
                       sweep vs exact-rational nearest-ties-up brute force.
  E8M0 block scale     reference KATs (quant/fp4_format.py:174-178) + exhaustive
                       sweep over every positive finite bf16 amax and fp32 edge
                       values vs exact rational arithmetic.
  pack/unpack          reference KAT [0,7,F,1,3] -> 70 1F 03 (:187-191) + round
                       trip.
  quantize_rows        composition of the above + dequant round-trip and
                       idempotence invariants + the C restatement.
  GEMM / MoE refs      brute force on tiny shapes and closed-form special cases
                       (identity-like codes, one-hot x, zero blocks, single
                       expert); beyond that float tolerance (parity unpinned
                       beyond tolerance, as the reference publishes no vectors).
  routing              torch.topk on the same fp32 probabilities plus a brute
                       force sort; indices bit-exact.
"""
