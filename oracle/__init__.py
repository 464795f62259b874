"""CPU oracle for the Qwen3.6-35B-A3B MoE block — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it. The product path (the HIP library behind the C-ABI
and its Python host layer) never imports, calls or falls back to anything here.

Modules
-------
ggml_quant   Q4_K / Q6_K super-block decoders and the 6-bit scale unpack, restated from the GGUF
             format as the reference reads it (tools/gguf_reader.py, tools/gguf_fast_dequant.py).
moe_oracle   The MoE block in the engine / policy-A form: correctly rounded R1, f32 softmax,
             torch.topk, f32 renorm, bf16 cast before the multiply, f32 experts, ascending-id
             combine, shared expert with its scalar sigmoid gate (speccheck/moe_ref.py,
             engine/m3_forward.py:430-476, engine/block_forward.py:614-681).
topk_model   A sequential model of torch's CPU topk for k*64 > n (libstdc++ nth_element +
             insertion sort of the first k-1), used to build tie fixtures and to pin the
             device's tie-order emulation against torch.topk.
configs      Seeded generators for BASELINE.json's configs (weights and inputs).

Pinning status (what checks each function; details in the test files):
  f16 decode            exhaustive over all 65,536 bit patterns vs numpy's IEEE conversion.
  q4k_scale_min         exhaustive over every (byte, byte) pair that feeds a field vs an
                        independent bit-level unpack, plus the reference's hand-worked vectors.
  dequant_q4k           reference KATs (d=dmin=1, all fields 63: q=0 -> -63, q=15 -> 882; the
                        element-33 sub-block witness = 945 with the min dropped), packer
                        round trips, f32-exactness proof checked against an f64 route.
  dequant_q6k           packer round trip against an independent expected-value route (the
                        reference has no hand-worked Q6_K KAT), exhaustive (sc, q) exactness.
  r1_logits             f64 brute force plus exact rational recompute at rounding midpoints.
  route / moe_block     invariants (weights sum to 1, descending order), closed forms
                        (one-hot x, W=0, E=K), brute-force f64 on tiny shapes.
  rmsnorm_a             closed form on constant rows, exact invariance under power-of-two
                        scaling (eps = 0), exact-rational scale on random rows, within 2 ulp of
                        torch's own f32 formula (the reference's arithmetic).
"""
