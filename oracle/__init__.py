"""CPU oracle for the batch-1 int4 decode path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or the timed CPU baseline). The product (flint_amd/) never imports it.

Contents (each function cites the reference file:line it restates):
  quant.py  - gpt-fast int4 group quantisation / dequantisation (engine/quantize.py)
  model.py  - gpt-fast forward on dequantised weights with the reference's bf16 rounding points
              (engine/model.py), NEOX RoPE, fp32 attention, greedy decode (engine/generate.py)

How each part is pinned (see tests/test_oracle.py):
  quant      closed-form invariants, brute force on tiny groups, and torch's independent CPU int4
             library kernel (aten::_weight_int4pack_mm_for_cpu) on the oracle's q / scales / zeros
  rope       NEOX-on-raw == interleaved-on-permuted identity (engine/scripts/convert_hf_checkpoint.py:75-81),
             pos=0 identity, rotation norm invariance
  attention  torch.nn.functional.scaled_dot_product_attention (library) in fp32; pos=0 known answer
  forward    golden vectors written by tests/golden/make_golden.py from the reference's own
             engine/model.py (imported in the build container only; fixtures committed)
"""
