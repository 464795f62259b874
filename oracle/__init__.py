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
lm_head_oracle  The untied lm_head's exact dot and the reference's acceptance band
             (prototype/lm_head/gate.py:214-240), and the Q8_0 decode the shared expert shares.

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
  route                 invariants (weights sum to 1, descending order), E = K; R5: the
                        weights equal an own bf16 RNE of the f32 renorm on the bit pattern and
                        reach the combine as bf16 (unit expert rows give them back exactly).
  R2 softmax            a near-equal-probability fixture (tests/r2_fixture.py): outside the rows
                        where distinct logits sit within 2 ulps, torch's softmax and an evaluation
                        with correctly rounded exps give the same ids; inside them the ids depend
                        on the exps' last bits (torch's CPU exps are within one ulp).
  experts_and_combine   one-hot rows: expert_raw[t, k] equals the closed form of expert
                        ids[t, k]; the neighbouring expert's closed form is far away.
  routed_combine        addends 2^24, 1, -2^24 whose f32 sum is 0 in ascending expert id and 1 in
                        rank order; weights reached by rank.
  moe_block             closed forms (identical experts, W = 0, one-hot x), brute-force f64 on
                        tiny shapes.
  from_device           split gate / up records stacked gate rows first.
  rmsnorm_a             closed form on constant rows, exact invariance under power-of-two
                        scaling (eps = 0), exact-rational scale on random rows, the association
                        (x * r) * w bit for bit with w not a power of two, within 3 ulp of
                        torch's own f32 formula (the reference's arithmetic).
"""
