"""GPU test of the allocation-free repair attention (ll_repair_attention_noalloc).

The entry keeps its split partial results in the library's device scratch
array instead of a caller workspace.  Two calls in a row -- the second with a
smaller plan, so the array still holds the first call's partials -- must give
bit for bit the output of ll_repair_attention with a workspace; a plan whose
partials exceed the array is rejected before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from legolink_amd import _native
from legolink_amd.repair_attention import RepairAttentionPlan

pytestmark = pytest.mark.gpu


def _spans(device, rng, *, requests: int, spans_per_request: int, span: int, gap: int, pool: int):
    spans = []
    for _ in range(requests):
        tokens = spans_per_request * (span + gap) + 16
        slots = torch.from_numpy(rng.permutation(pool)[:tokens].astype(np.int64)).to(device)
        for index in range(spans_per_request):
            start = gap + index * (span + gap)
            spans.append((slots, start, start + span))
    return spans


def _both_outputs(device, spans, *, split_tokens: int, seed: int, q_heads=28, kv_heads=4, head_dim=128,
                  pool=8192):
    generator = torch.Generator(device=device).manual_seed(seed)
    key = torch.randn(pool, kv_heads, head_dim, device=device, generator=generator).to(torch.bfloat16)
    value = torch.randn(pool, kv_heads, head_dim, device=device, generator=generator).to(torch.bfloat16)
    common = dict(num_q_heads=q_heads, num_kv_heads=kv_heads, head_dim=head_dim, pool_size=pool,
                  split_tokens=split_tokens)
    with_workspace = RepairAttentionPlan(spans, **common)
    without = RepairAttentionPlan(spans, allocation_free=True, **common)
    assert without.workspace is None
    assert with_workspace.info == without.info
    query = torch.randn(with_workspace.num_queries, q_heads, head_dim, device=device,
                        generator=generator).to(torch.bfloat16)
    want = with_workspace.run(query, key, value)
    got = without.run(query, key, value)
    torch.cuda.synchronize(device)
    return with_workspace.info, got, want


def test_allocation_free_attention_matches_the_workspace_entry(gpu_device):
    rng = np.random.default_rng(20260824)
    scratch = _native.repair_scratch_bytes()
    assert scratch == 64 << 20
    # First call: 3 requests x 4 spans, forced 256-key chunks (many partials).
    big = _spans(gpu_device, rng, requests=3, spans_per_request=4, span=16, gap=600, pool=8192)
    print("allocation-free call 1: 12 spans, split 256", flush=True)
    info, got, want = _both_outputs(gpu_device, big, split_tokens=256, seed=1)
    assert info["num_combine"] > 0 and info["workspace_items"] > 20
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # Second call, smaller: the scratch still holds the first call's partials.
    small = _spans(gpu_device, rng, requests=1, spans_per_request=2, span=9, gap=300, pool=8192)
    print("allocation-free call 2: 2 spans, split 128", flush=True)
    info2, got, want = _both_outputs(gpu_device, small, split_tokens=128, seed=2)
    assert 0 < info2["workspace_items"] < info["workspace_items"]
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_allocation_free_attention_without_split_items(gpu_device):
    rng = np.random.default_rng(5)
    spans = _spans(gpu_device, rng, requests=2, spans_per_request=2, span=8, gap=40, pool=4096)
    info, got, want = _both_outputs(gpu_device, spans, split_tokens=0, seed=3, pool=4096)
    assert info["num_combine"] == 0
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_allocation_free_attention_rejects_plans_beyond_the_scratch(gpu_device):
    """Checked on the host before any launch: more than 567 partials of 28
    heads at head dim 128 (4,224 bytes per head) need more than 64 MiB."""

    rng = np.random.default_rng(9)
    spans = _spans(gpu_device, rng, requests=1, spans_per_request=40, span=16, gap=260, pool=16384)
    plan = RepairAttentionPlan(spans, num_q_heads=28, num_kv_heads=4, head_dim=128, pool_size=16384,
                               split_tokens=64, allocation_free=True)
    needed = plan.info["workspace_items"] * 28 * (8 * 128 + 32) * 4
    assert needed > _native.repair_scratch_bytes()
    key = torch.zeros(16384, 4, 128, dtype=torch.bfloat16, device=gpu_device)
    query = torch.zeros(plan.num_queries, 28, 128, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(_native.NativeCallError, match="scratch array holds"):
        plan.run(query, key, key)
