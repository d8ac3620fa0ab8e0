"""The harness's acceptance check at the five benchmark configurations:
``verify`` (HIP card against the spec's reference) and ``verify_parity`` (HIP
card against the reference card, same inputs) at full size, through the
reference's own entry points (src/xkernels/verify.py:169-279, 340-437) with
``shapes=``.

  C1  int4 W4A16   M=16,   E=8,   N=1024, K=2048, top_k=2
  C2  int4 W4A16   M=64,   E=48,  N=4096, K=7168, top_k=8   (decode)
  C3  align        M=16384, top_k=8, E=48, block 16
      sum_reduce   [8192, 8, 7168] bf16
  C4  mxfp4        M=48, E=256, hidden 4096, ispp 512, top_k=6
  C5  int4 W4A16   M=4096, E=48,  N=4096, K=7168, top_k=8   (prefill)

The harness draws its own seeded inputs (registry/input_gen.py: uniform routing
with possible repeats per token); the Zipf-routed variants of C3 and C5 are
covered by the direct parity tests. C4 runs at the input scale of the
reference's own C4-shaped test (A x 0.1, tests/test_moe_mxfp4.py:62-68
upstream): at A ~ N(0, 1) the gate/up sums reach ~50 and their bf16 rounding
(ulp 0.25) alone moves outputs by more than the elementwise 2e-2, for any two
implementations that sum in different orders; that case is checked in
tests/test_gpu_mxfp4.py against the output's own scale.
"""
from __future__ import annotations

import pytest

from xkernels_amd import verify, verify_parity

pytestmark = pytest.mark.gpu

CONFIGS = [
    ("C1", "moe_int4_w4a16", dict(dtype="bf16", M=16, K=2048, N=1024, E=8, top_k=2)),
    ("C2", "moe_int4_w4a16", dict(dtype="bf16", M=64, K=7168, N=4096, E=48, top_k=8)),
    ("C3", "moe_align_block_size", dict(dtype="int32", M=16384, top_k=8, num_experts=48, block_size=16)),
    ("C3", "moe_sum_reduce", dict(dtype="bf16", M=8192, top_k=8, H=7168)),
    ("C4", "moe_mxfp4", dict(dtype="bf16", M=48, E=256, hidden=4096, ispp=512, top_k=6, a_scale=0.1)),
    ("C5", "moe_int4_w4a16", dict(dtype="bf16", M=4096, K=7168, N=4096, E=48, top_k=8)),
]
IDS = [f"{c}-{op}" for c, op, _ in CONFIGS]


@pytest.mark.parametrize("cfg,op,point", CONFIGS, ids=IDS)
def test_verify_at_config(cfg, op, point, dev):
    print(f"verify {cfg} {op} {point}", flush=True)
    r = verify(f"{op}.hip@1.0.0", arch="amd_cdna4", shapes=[point])
    assert r["compiled"], r["artifacts"]
    assert r["correctness"]["passed"], r["correctness"]
    assert r["determinism_check"]


@pytest.mark.parametrize("cfg,op,point", CONFIGS, ids=IDS)
def test_verify_parity_at_config(cfg, op, point, dev):
    print(f"verify_parity {cfg} {op} {point}", flush=True)
    r = verify_parity(f"{op}@1.0.0", archs=["amd_cdna4"], shapes=[point])
    assert r["device"] == "cuda"
    assert r["n_runnable"] == 2, r["errors"]
    assert r["agree"] is True, r["diverging"]
