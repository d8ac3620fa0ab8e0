"""moe_align_block_size on the GPU: bit-exact against the oracle (align.py:34-70).

Mirrors the reference's tests/test_moe_align_block_size.py cases (random,
skewed, single expert, truncate=False fixed shape) plus the BASELINE config
(M=16384, top_k=8, E=48, bs=16, Zipf 1.1), the grid path (>8192 slots or >512
experts), EP drops and ids outside [0, E).
"""
from __future__ import annotations

import pytest
import torch

from oracle import c_oracle
from oracle.torch_ref import moe_align_block_size_ref
from tests._helpers import zipf_topk
from xkernels_amd import Backend, MoeAlignWorkspace, moe_align_block_size

pytestmark = pytest.mark.gpu


def _ids(M, top_k, E, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, E, (M, top_k), generator=g, dtype=torch.int32)


def _check(ids_cpu, bs, E, truncate, dev):
    got = moe_align_block_size(ids_cpu.to(dev), bs, E, backend=Backend.HIP, truncate=truncate)
    ref = moe_align_block_size_ref(ids_cpu, bs, E, truncate=truncate)
    for name, g, r in zip(("sorted_token_ids", "expert_ids", "num_post"), got, ref):
        assert g.dtype == torch.int32, name
        assert torch.equal(g.cpu(), r), f"{name} mismatch (M*k={ids_cpu.numel()}, E={E}, bs={bs}, truncate={truncate})"


@pytest.mark.parametrize("M,top_k,E,bs", [(8, 2, 4, 4), (16, 8, 48, 16), (1, 8, 48, 16), (32, 4, 8, 8),
                                          (7, 3, 5, 4), (64, 2, 16, 32), (64, 8, 48, 16), (37, 4, 8, 16),
                                          (16, 1, 4, 8), (48, 6, 256, 16), (512, 8, 48, 64)])
@pytest.mark.parametrize("truncate", [True, False])
def test_matches_oracle(M, top_k, E, bs, truncate, dev):
    _check(_ids(M, top_k, E), bs, E, truncate, dev)


@pytest.mark.parametrize("seed", range(8))
def test_randomized_skewed(seed, dev):
    g = torch.Generator().manual_seed(seed)
    M = int(torch.randint(1, 40, (1,), generator=g))
    top_k = int(torch.randint(1, 9, (1,), generator=g))
    E = int(torch.randint(2, 33, (1,), generator=g))
    bs = int(2 ** torch.randint(2, 6, (1,), generator=g))
    ids = torch.randn(M, top_k, E, generator=g).argmax(-1).to(torch.int32)
    _check(ids, bs, E, True, dev)
    _check(ids, bs, E, False, dev)


def test_single_expert_all_tokens(dev):
    _check(torch.zeros((10, 4), dtype=torch.int32), 8, 6, True, dev)


@pytest.mark.parametrize("M,top_k,E,bs,s", [(16384, 8, 48, 16, 1.1), (4096, 8, 48, 64, 1.2),
                                            (2000, 8, 48, 16, 1.1), (300, 4, 600, 16, 0.5)])
def test_grid_path_zipf(M, top_k, E, bs, s, dev):
    ids = zipf_topk(M, top_k, E, s, seed=11)
    _check(ids, bs, E, True, dev)
    _check(ids, bs, E, False, dev)
    # independent C restatement agrees too (fixed-shape form)
    c = c_oracle.align(ids, bs, E)
    got = moe_align_block_size(ids.to(dev), bs, E, backend=Backend.HIP, truncate=False)
    for g, r in zip(got, c):
        assert torch.equal(g.cpu(), r)


def test_empty_routing(dev):
    ids = torch.zeros((0, 8), dtype=torch.int32)
    _check(ids, 16, 48, True, dev)
    _check(ids, 16, 48, False, dev)


def test_out_of_range_ids_are_not_placed(dev):
    ids = _ids(20, 4, 10)
    ids[0, 0] = 10   # == num_experts: counted nowhere, never placed
    ids[3, 2] = 12
    _check(ids, 4, 10, True, dev)
    _check(ids, 4, 10, False, dev)


def test_workspace_reuse_smaller_M(dev):
    ws = MoeAlignWorkspace.allocate(64, 8, 48, 16, device=dev)
    addr = ws.sorted_ids.data_ptr()
    for M in (64, 16):
        ids = _ids(M, 8, 48, seed=M)
        got = moe_align_block_size(ids.to(dev), 16, 48, backend=Backend.HIP, truncate=False, workspace=ws)
        ref = moe_align_block_size_ref(ids, 16, 48, truncate=False)
        for g, r in zip(got, ref):
            assert torch.equal(g.cpu(), r)
        assert got[0].data_ptr() == addr


def test_cpu_tensor_is_rejected():
    with pytest.raises(RuntimeError, match="device tensors"):
        moe_align_block_size(torch.zeros((2, 2), dtype=torch.int32), 4, 4, backend=Backend.HIP)
