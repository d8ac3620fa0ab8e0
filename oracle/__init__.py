"""CPU oracle of the xkernels quantized fused-MoE path — TEST INFRASTRUCTURE.

``torch_ref``: pure-torch restatement of the reference backend (also the
REFERENCE backend the test harness registers). ``c_oracle``: independent
plain-C restatement (moe_oracle.c, built by ``make -C oracle``) used as a second
oracle and as the benchmark's CPU baseline. Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline may import this package; the product package
``xkernels_amd`` never does.

Parity status per function (pinning checks live in tests/test_oracle.py):
  align (torch + C)        pinned: brute-force stable sort on tiny inputs,
                           structural invariants, torch == C bit-exact
  dequant_w4a16            pinned: closed-form known answers (nibble order,
                           -8 offset, group scale broadcast, bf16 RNE)
  moe_w4a16_ref            pinned: literal per-(m, j) loop, dense matmul of
                           generator-chosen weights, linearity / EP partition
  moe_sum_reduce_ref       pinned: one-hot weights select rows exactly, closed
                           form on integer-valued inputs
  dequant_mxfp4            pinned: e2m1 values rebuilt from sign/exponent/
                           mantissa bit fields, e8m0 special codes
  moe_mxfp4_ref            pinned: torch == C restatement, single-expert dense
                           recomputation, EP partition, limit disable
The torch operations the reference itself relies on (argsort, bincount,
matmul, silu) are third-party arithmetic (torch >= 2.1, unpinned upstream);
their use here is anchored by the checks above.
"""
