"""Oracle for the fused RMSNorm + W4A16 MoE path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this package, and only as the checker (or
as the timed CPU baseline). The product (the package and its HIP library) never
imports, links or runs anything here.

- moe_oracle.py : numpy restatement of the reference's dtype chain.
- oracle_c.c    : C restatement of the bit-exact pieces (fixed-order fmaf
                  combine, counting-sort routing), built by the Makefile into
                  liboracle.so and loaded through ctypes (oracle_c.py).
- cpu_baseline.py : the reference CPU path in torch eager, timed by bench.py.

Parity status per function (how each one is pinned):
- rmsnorm      : pinned (stock transformers DiffusionGemmaRMSNorm, closed forms).
- quantize_w4 / dequant_w4 : pinned (hand-computed known answers, exactness).
- moe_align    : pinned (hand-computed known answer, brute force, C counting sort).
- act_fp32     : pinned (float64 closed forms of tanh-GELU and SiLU).
- gateup_act / down / moe_forward : pinned (dense F.linear reduction, brute
  force loops, stock DiffusionGemmaTextExperts.forward on dequantised weights).
- combine_fma / orc_combine : pinned (identity gather, exact mean, fmaf).
"""
