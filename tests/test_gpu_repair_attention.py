"""GPU parity of the sparse repair attention kernel against the fp64 oracle of
the reference's gqa_attention over logical_causal_mask, and against a plain
torch fp32 restatement.

Tolerance, elementwise: |got - ref| <= 2^-7 * (sum_j w_j |v_j| + |ref|) + 1e-5,
where w are the softmax weights.  The kernel rounds each probability to bf16
for the value product (relative error <= 2^-8, so the output moves by at most
2^-8 * sum_j w_j |v_j|), a split range's partial output O / l to bf16 (the
merge is a convex combination of the partials: at most 2^-9 * sum_j w_j |v_j|
more) and the output to bf16 (<= 2^-9 * |ref|); the bound is above the sum.  fp16 inputs round to fp16 instead (2^-11) and keep the same
bound.  The reference's own FlashInfer check is atol = rtol = 3e-2
(tests/pic/test_sparse_attention_reference.py:103).  Short KVs, a sharp
softmax (scale 1) and zero queries make an off-by-one mask or a dropped key
(an output change of w_j |v_j - ref|, >= 2.5e-2 there) visible above it.
"""

from __future__ import annotations

import math
import zlib

import numpy as np
import pytest
import torch

from legolink_amd.repair_attention import RepairAttentionPlan, SparseRepairAttentionError, sparse_repair_attention
from oracle import attention_oracle as ao
from tests.gpu_helpers import report

pytestmark = pytest.mark.gpu


def _bf16(shape, generator, device, scale=1.0, dtype=torch.bfloat16):
    return (torch.randn(shape, generator=generator, device=device) * scale).to(dtype)


def _torch_fp32(query, key_rows, value_rows, visible, scale):
    """Plain fp32 torch attention on the CPU (GQA by head // group)."""

    q = query.float().cpu()
    k = key_rows.float().cpu()
    v = value_rows.float().cpu()
    group = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1)
    scores = torch.einsum("qhd,khd->hqk", q, k) * scale
    scores = scores.masked_fill(~torch.from_numpy(visible)[None], float("-inf"))
    return torch.einsum("hqk,khd->qhd", torch.softmax(scores, dim=-1), v).numpy()


def _check(plan_spans, query, key_pool, value_pool, got, scale):
    q_np = query.float().cpu().numpy()
    k_np = key_pool.float().cpu().numpy()
    v_np = value_pool.float().cpu().numpy()
    got_np = got.float().cpu().numpy()
    cursor = 0
    worst = 0.0
    for slots, start, end in plan_spans:
        n = end - start
        slots_np = slots.cpu().numpy()
        q_part = q_np[cursor : cursor + n]
        want = ao.repair_attention(q_part, k_np, v_np, slots_np, start, end, scale=scale)
        magnitude = ao.repair_attention(q_part, k_np, np.abs(v_np), slots_np, start, end, scale=scale)
        bound = 2.0 ** -7 * (magnitude + np.abs(want)) + 1e-5
        valid = (slots_np[:end] >= 0) & (slots_np[:end] < k_np.shape[0])
        safe = torch.from_numpy(np.where(valid, slots_np[:end], 0))
        visible = ao.logical_causal_mask(np.arange(start, end), np.arange(end)) & valid[None]
        keep = torch.from_numpy(valid)[:, None, None]
        fp32 = _torch_fp32(query[cursor : cursor + n], torch.where(keep, key_pool.cpu()[safe], 0),
                           torch.where(keep, value_pool.cpu()[safe], 0), visible, scale)
        part = got_np[cursor : cursor + n]
        err = np.abs(part - want)
        worst = max(worst, float((err / bound).max()))
        bad = err > bound
        assert not bad.any(), f"span [{start}, {end}): {int(bad.sum())} elements off, max err {err.max():.3g}"
        # A query that sees no valid key (its only keys' slots invalid) outputs
        # zeros, as the oracle defines it; torch's softmax over an all -inf row
        # is NaN, so the fp32 restatement is compared on the other rows.
        seen = visible.any(axis=1)
        assert (part[~seen] == 0).all()
        assert (np.abs(part - fp32) <= bound + 2.0 ** -8 * np.abs(fp32))[seen].all()
        cursor += n
    report(f"largest error / bound vs fp64: {worst:.3f}")


CASES = [
    # name, q heads, kv heads, head dim, spans (start, end), pool slots, split tokens, scale
    ("qwen7b_one_span", 28, 4, 128, [(100, 116)], 4096, 0, None),
    ("partial_tiles", 28, 4, 128, [(0, 1), (5, 22), (40, 73)], 4096, 0, None),
    ("long_kv_forced_splits", 28, 4, 128, [(9000, 9020)], 16384, 512, None),
    ("seams_auto_split", 28, 4, 128, [(s, s + 16) for s in range(1024, 16384, 1024)], 32768, 0, None),
    ("group8_head_dim64", 16, 2, 64, [(30, 50), (200, 201)], 2048, 0, None),
    ("group1", 8, 8, 128, [(10, 26)], 2048, 0, None),
    ("sharp_softmax", 28, 4, 128, [(3, 40), (300, 333)], 4096, 128, 1.0),
    # GQA ratios above 8: windows of 16 pairs hold one tile or part of one;
    # from 16 heads up each tile's heads take several windows.
    ("group12", 24, 2, 128, [(50, 70), (400, 416)], 2048, 0, None),
    ("mqa_group32", 32, 1, 128, [(100, 133)], 2048, 256, None),
    ("mqa_group71_head_dim64", 71, 1, 64, [(20, 37), (900, 905)], 2048, 0, None),
    # Head dim 256: 8 (tile, head) pairs per workgroup, so a window of 16
    # pairs takes two workgroups, and 20 heads of one tile take two windows
    # (16 and 4).
    ("head_dim256_group2", 8, 4, 256, [(10, 40), (600, 616)], 2048, 0, None),
    ("head_dim256_group7_split", 28, 4, 256, [(1500, 1520)], 4096, 512, None),
    ("head_dim256_mqa_group20", 20, 1, 256, [(300, 345)], 2048, 0, None),
    # Small groups: a window of 16 pairs holds 16 / G tiles (MHA: 16).  At head
    # dim 256 (8 pairs per workgroup) a window is split over two workgroups.
    ("mha_thirteen_tiles", 8, 8, 128, [(100, 300)], 4096, 0, None),
    ("mha_tiles_with_forced_splits", 4, 4, 64, [(40, 60), (600, 900)], 4096, 256, None),
    ("group2_eight_tiles", 16, 8, 128, [(10, 150)], 2048, 0, None),
    ("head_dim256_mha_tile_split", 4, 4, 256, [(50, 250)], 4096, 0, None),
    ("head_dim256_group3_tile_split", 12, 4, 256, [(30, 130)], 2048, 512, None),
    # Groups that do not divide 16: windows start and end inside tiles (7
    # heads: 16-pair windows over 10 tiles; 5 heads with contiguous spans and
    # forced splits; head dim 256, two workgroups per window; 3 heads over
    # short spans sharing tiles).
    ("group7_windows_cross_tiles", 28, 4, 128, [(200, 360)], 4096, 0, None),
    ("group5_windows_cross_tiles_split", 20, 4, 128, [(1000, 1100), (1100, 1164)], 4096, 256, None),
    ("head_dim256_group7_windows", 28, 4, 256, [(300, 400)], 4096, 0, None),
    ("group3_short_spans_head_dim64", 12, 4, 64, [(s, s + 8) for s in range(100, 2000, 150)], 4096, 0, None),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_repair_attention_matches_oracle(gpu_device, case):
    name, hq, hkv, dim, spans, pool, split, scale = case
    report(f"case {name}: hq={hq} hkv={hkv} d={dim} spans={spans[:3]}... pool={pool} split={split}")
    generator = torch.Generator(device=gpu_device).manual_seed(zlib.crc32(name.encode()) % 1000)
    key_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    value_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    length = max(end for _, end in spans)
    slots = torch.randperm(pool, generator=generator, device=gpu_device)[:length]
    plan_spans = [(slots, start, end) for start, end in spans]
    plan = RepairAttentionPlan(plan_spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim,
                               pool_size=pool, split_tokens=split)
    report(f"plan {plan.info}")
    query = _bf16((plan.num_queries, hq, dim), generator, gpu_device)
    use_scale = scale if scale is not None else 1.0 / math.sqrt(dim)
    got = plan.run(query, key_pool, value_pool, scale=scale)
    torch.cuda.synchronize(gpu_device)
    _check(plan_spans, query, key_pool, value_pool, got, use_scale)


FP16_CASES = [c for c in CASES if c[0] in ("qwen7b_one_span", "long_kv_forced_splits", "seams_auto_split",
                                           "group8_head_dim64", "head_dim256_group7_split")]


@pytest.mark.parametrize("case", FP16_CASES, ids=[c[0] for c in FP16_CASES])
def test_fp16_matches_oracle(gpu_device, case):
    """The reference takes fp16 or bf16 Q/K/V (flashinfer_sparse_repair.py:977-980)."""

    name, hq, hkv, dim, spans, pool, split, scale = case
    report(f"fp16 case {name}")
    generator = torch.Generator(device=gpu_device).manual_seed(zlib.crc32(name.encode()) % 1000 + 1)
    key_pool = _bf16((pool, hkv, dim), generator, gpu_device, dtype=torch.float16)
    value_pool = _bf16((pool, hkv, dim), generator, gpu_device, dtype=torch.float16)
    length = max(end for _, end in spans)
    slots = torch.randperm(pool, generator=generator, device=gpu_device)[:length]
    plan_spans = [(slots, start, end) for start, end in spans]
    plan = RepairAttentionPlan(plan_spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim,
                               pool_size=pool, split_tokens=split)
    query = _bf16((plan.num_queries, hq, dim), generator, gpu_device, dtype=torch.float16)
    got = plan.run(query, key_pool, value_pool, scale=scale)
    torch.cuda.synchronize(gpu_device)
    assert got.dtype == torch.float16
    _check(plan_spans, query, key_pool, value_pool, got, scale if scale is not None else 1.0 / math.sqrt(dim))


@pytest.mark.parametrize("seed", range(96))
def test_random_configurations(gpu_device, seed):
    """Seeded random shapes: GQA group, head dim, dtype, slot dtype, several
    requests and spans (partial tiles, seams near chunk edges, long spans whose
    work windows cross many tiles), chunk length, scale and a few invalid
    slots; checked against the fp64 oracle."""

    rng = np.random.default_rng(1000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 11, 12, 15, 16, 20]))
    hq = hkv * group
    dim = int(rng.choice([64, 128, 256]))
    dtype = torch.float16 if rng.random() < 0.4 else torch.bfloat16
    pool = int(rng.integers(2048, 8192))
    split = int(rng.choice([0, 64, 128, 512, 1024]))
    scale = float(rng.choice([1.0 / math.sqrt(dim), 0.5, 1.0]))
    generator = torch.Generator(device=gpu_device).manual_seed(seed)
    key_pool = _bf16((pool, hkv, dim), generator, gpu_device, dtype=dtype)
    value_pool = _bf16((pool, hkv, dim), generator, gpu_device, dtype=dtype)
    order = torch.randperm(pool, generator=generator, device=gpu_device)
    spans, cursor = [], 0
    for _ in range(int(rng.integers(1, 4))):
        length = min(int(rng.integers(20, 3000)), pool - cursor)
        if length < 20:
            break
        slots = order[cursor : cursor + length].clone()
        cursor += length
        if rng.random() < 0.5:
            slots = slots.to(torch.int32)
        if rng.random() < 0.3:
            slots[int(rng.integers(0, length))] = -1
        for _ in range(int(rng.integers(1, 4))):
            end = int(rng.integers(1, length + 1))
            longest = 300 if rng.random() < 0.25 else 40
            start = max(0, end - int(rng.integers(1, longest)))
            spans.append((slots, start, end))
    report(f"seed {seed}: hq={hq} hkv={hkv} d={dim} {dtype} split={split} scale={scale:.3f} "
           f"spans={[(s, e) for _, s, e in spans]}")
    plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim, split_tokens=split,
                               validate=False)
    query = _bf16((plan.num_queries, hq, dim), generator, gpu_device, dtype=dtype)
    got = plan.run(query, key_pool, value_pool, scale=scale)
    torch.cuda.synchronize(gpu_device)
    _check(spans, query, key_pool, value_pool, got, scale)


@pytest.mark.parametrize("seed", range(12))
def test_random_long_requests(gpu_device, seed):
    """Seeded random long requests (8,000-24,000 keys), so that work items
    cross one or more slot-list refills (every 7,680 keys): chunk lengths
    beyond the refill size or automatic, invalid slots on refill edges, GQA
    groups 1-8, head dims 64 and 128."""

    rng = np.random.default_rng(5000 + seed)
    hkv = int(rng.choice([1, 2]))
    group = int(rng.choice([1, 3, 4, 7, 8]))
    hq = hkv * group
    dim = int(rng.choice([64, 128]))
    dtype = torch.float16 if rng.random() < 0.3 else torch.bfloat16
    length = int(rng.integers(8000, 24000))
    pool = length + int(rng.integers(16, 2000))
    split = int(rng.choice([0, 0, 8960, 16384, 24576]))
    generator = torch.Generator(device=gpu_device).manual_seed(seed + 77)
    key_pool = _bf16((pool, hkv, dim), generator, gpu_device, dtype=dtype)
    value_pool = _bf16((pool, hkv, dim), generator, gpu_device, dtype=dtype)
    slots = torch.randperm(pool, generator=generator, device=gpu_device)[:length].clone()
    for edge in range(7680, length, 7680):
        if rng.random() < 0.5:
            slots[edge - int(rng.integers(0, 2))] = -1
    if rng.random() < 0.5:
        slots = slots.to(torch.int32)
    spans = []
    for _ in range(int(rng.integers(1, 3))):
        end = int(rng.integers(length // 3, length + 1))
        spans.append((slots, max(0, end - int(rng.integers(1, 24))), end))
    report(f"long seed {seed}: hq={hq} hkv={hkv} d={dim} {dtype} length={length} split={split} "
           f"spans={[(s, e) for _, s, e in spans]}")
    plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim, split_tokens=split,
                               validate=False)
    scale = 1.0 / math.sqrt(dim)
    query = _bf16((plan.num_queries, hq, dim), generator, gpu_device, dtype=dtype)
    got = plan.run(query, key_pool, value_pool, scale=scale)
    torch.cuda.synchronize(gpu_device)
    _check(spans, query, key_pool, value_pool, got, scale)


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("split", [192, 704, 2112, 4160, 7680])
def test_chunk_lengths_of_the_plan_search(gpu_device, split, dim):
    """Key chunks of the lengths the plan's fine search picks (multiples of 64
    that are not powers of two) up to 7,680 keys, whose slot list
    fills the LDS the ring leaves: spans of an 8,000-token request ending
    just before, at and after chunk edges, GQA 7/1 and a 16-query span."""

    generator = torch.Generator(device=gpu_device).manual_seed(split + dim)
    pool, length = 9000, 8000
    key_pool = _bf16((pool, 1, dim), generator, gpu_device)
    value_pool = _bf16((pool, 1, dim), generator, gpu_device)
    slots = torch.randperm(pool, generator=generator, device=gpu_device)[:length].clone()
    ends = sorted({min(length, max(16, e)) for e in (split - 1, split, split + 1, 2 * split + 33, length)})
    spans = [(slots, end - 16, end) for end in ends]
    report(f"chunk {split}, head dim {dim}: spans {[(s, e) for _, s, e in spans]}")
    plan = RepairAttentionPlan(spans, num_q_heads=7, num_kv_heads=1, head_dim=dim, split_tokens=split,
                               pool_size=pool)
    assert plan.info["split_tokens"] == split
    assert plan.info["workspace_items"] > 0  # the longest spans are split
    query = _bf16((plan.num_queries, 7, dim), generator, gpu_device)
    scale = 1.0 / math.sqrt(dim)
    got = plan.run(query, key_pool, value_pool, scale=scale)
    torch.cuda.synchronize(gpu_device)
    _check(spans, query, key_pool, value_pool, got, scale)


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("split", [7744, 15360, 20032])
def test_items_longer_than_one_slot_list(gpu_device, split, dim):
    """Work items over more keys than the slot list holds (7,680): the
    workgroup refills it every 7,680 keys, carrying the softmax state, so an
    item may span a whole request (20,032: every item whole).  A
    20,000-token request with invalid slots on both sides of each refill
    boundary; spans ending just before, at and after the boundaries."""

    generator = torch.Generator(device=gpu_device).manual_seed(split + dim + 5)
    pool, length = 21000, 20000
    key_pool = _bf16((pool, 1, dim), generator, gpu_device)
    value_pool = _bf16((pool, 1, dim), generator, gpu_device)
    slots = torch.randperm(pool, generator=generator, device=gpu_device)[:length].clone()
    for edge in (7680, 15360):
        slots[edge - 1] = -1
        slots[edge] = pool + 3  # outside the pool: an invisible key too
    ends = [7679, 7680, 7681, 15359, 15361, 19000, 20000]
    spans = [(slots, end - 16, end) for end in ends] + [(slots, 7600, 7700)]
    report(f"long items, split {split}, head dim {dim}: spans {[(s, e) for _, s, e in spans]}")
    plan = RepairAttentionPlan(spans, num_q_heads=7, num_kv_heads=1, head_dim=dim, split_tokens=split,
                               validate=False)
    assert plan.info["split_tokens"] == split
    if split >= length:
        assert plan.info["workspace_items"] == 0, plan.info  # whole items, no combine
    query = _bf16((plan.num_queries, 7, dim), generator, gpu_device)
    scale = 1.0 / math.sqrt(dim)
    got = plan.run(query, key_pool, value_pool, scale=scale)
    torch.cuda.synchronize(gpu_device)
    _check(spans, query, key_pool, value_pool, got, scale)


def test_dtype_checks_follow_the_reference(gpu_device):
    slots = torch.arange(64, device=gpu_device)
    plan = RepairAttentionPlan([(slots, 10, 26)], num_q_heads=8, num_kv_heads=2, head_dim=64)
    kv16 = torch.zeros((64, 2, 64), dtype=torch.float16, device=gpu_device)
    q = torch.zeros((16, 8, 64), dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(SparseRepairAttentionError, match="dtypes must match"):
        plan.run(q, kv16, kv16)
    with pytest.raises(SparseRepairAttentionError, match="unsupported Q dtype"):
        plan.run(q.float(), kv16.float(), kv16.float())


def test_two_requests_in_one_plan_with_int32_slots(gpu_device):
    generator = torch.Generator(device=gpu_device).manual_seed(2)
    hq, hkv, dim, pool = 28, 4, 128, 8192
    key_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    value_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    order = torch.randperm(pool, generator=generator, device=gpu_device)
    first = order[:700]
    second = order[700:1100].to(torch.int32)
    spans = [(first, 500, 516), (second, 20, 45), (first, 680, 700), (second, 399, 400)]
    plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim, pool_size=pool)
    query = _bf16((plan.num_queries, hq, dim), generator, gpu_device)
    got = plan.run(query, key_pool, value_pool)
    torch.cuda.synchronize(gpu_device)
    _check(spans, query, key_pool, value_pool, got, 1.0 / math.sqrt(dim))


def test_invalid_slots_are_invisible_keys(gpu_device):
    generator = torch.Generator(device=gpu_device).manual_seed(3)
    hq, hkv, dim, pool = 28, 4, 128, 1024
    key_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    value_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    # Slot 0 is never visible and holds Inf and NaN: tokens without a valid slot
    # (and the padding of the last key tile) must not reach the output.
    slots = (torch.randperm(pool - 1, generator=generator, device=gpu_device)[:200] + 1).clone()
    slots[[3, 77, 150]] = torch.tensor([-1, pool, pool + 50], device=gpu_device)
    key_pool[0] = float("inf")
    value_pool[0] = float("nan")
    spans = [(slots, 140, 180)]
    with pytest.raises(SparseRepairAttentionError, match="invalid KV slots"):
        RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim, pool_size=pool)
    plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim, validate=False)
    query = _bf16((plan.num_queries, hq, dim), generator, gpu_device)
    got = plan.run(query, key_pool, value_pool)
    torch.cuda.synchronize(gpu_device)
    _check(spans, query, key_pool, value_pool, got, 1.0 / math.sqrt(dim))


def test_zero_queries_average_the_visible_values(gpu_device):
    """q = 0 gives equal weights: output row i is the mean of the values at
    positions 0..start + i -- exact up to the final bf16 rounding."""

    generator = torch.Generator(device=gpu_device).manual_seed(4)
    hq, hkv, dim, pool = 28, 4, 128, 2048
    key_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    value_pool = _bf16((pool, hkv, dim), generator, gpu_device)
    slots = torch.randperm(pool, generator=generator, device=gpu_device)[:300]
    start, end = 250, 290
    query = torch.zeros((end - start, hq, dim), dtype=torch.bfloat16, device=gpu_device)
    got = sparse_repair_attention(query, key_pool, value_pool, slots, repair_start=start, repair_end=end)
    torch.cuda.synchronize(gpu_device)
    values = value_pool.float().cpu().numpy()[slots.cpu().numpy()]
    for i in range(end - start):
        mean = values[: start + i + 1].mean(axis=0)                      # [hkv, dim]
        want = np.repeat(mean, hq // hkv, axis=0)
        assert np.allclose(got[i].float().cpu().numpy(), want, rtol=2 ** -8, atol=1e-6), i


def test_one_plan_serves_every_layer(gpu_device):
    generator = torch.Generator(device=gpu_device).manual_seed(6)
    hq, hkv, dim, pool = 28, 4, 128, 4096
    slots = torch.randperm(pool, generator=generator, device=gpu_device)[:2500]
    spans = [(slots, 1000, 1016), (slots, 2000, 2016), (slots, 2400, 2450)]
    plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim, pool_size=pool)
    for layer in range(3):
        key_pool = _bf16((pool, hkv, dim), generator, gpu_device)
        value_pool = _bf16((pool, hkv, dim), generator, gpu_device)
        query = _bf16((plan.num_queries, hq, dim), generator, gpu_device)
        got = plan.run(query, key_pool, value_pool)
        torch.cuda.synchronize(gpu_device)
        _check(spans, query, key_pool, value_pool, got, 1.0 / math.sqrt(dim))


@pytest.mark.parametrize("dim,pool", [(128, (1 << 22) - 1), (128, 4_500_000), (256, (1 << 21) - 1),
                                      (256, 2_200_000), (64, (1 << 23) - 1), (64, 9_000_000)],
                         ids=["d128_top_rows_of_a_4gib_buffer", "d128_beyond_4gib", "d256_top_rows_of_a_4gib_buffer",
                              "d256_beyond_4gib", "d64_top_rows_of_a_4gib_buffer", "d64_beyond_4gib"])
def test_pools_at_and_beyond_32_bit_row_offsets(gpu_device, dim, pool):
    """K and V buffers of up to 4 GiB (4 KV heads: 4,194,303 slots of 1 KiB
    rows at head dim 128, 2,097,151 at 256, 8,388,607 at 64) are gathered
    with 32-bit byte offsets, larger ones with 64-bit addresses.  Slots at
    the top of each pool give the same output, bit for bit, as the same rows
    gathered from a small pool, and match the oracle."""

    generator = torch.Generator(device=gpu_device).manual_seed(8)
    hq, hkv = 28, 4
    key_pool = torch.empty((pool, hkv, dim), dtype=torch.bfloat16, device=gpu_device)
    value_pool = torch.empty_like(key_pool)
    # 3,000 distinct slots: most in the pool's top 64 Ki rows (past 4 GiB in
    # the larger pool), a few at the bottom.
    top = pool - 1 - torch.randperm(1 << 16, generator=generator, device=gpu_device)[:2900]
    slots = torch.cat([top, torch.randperm(1 << 12, generator=generator, device=gpu_device)[:100]])
    slots = slots[torch.randperm(slots.numel(), generator=generator, device=gpu_device)]
    rows_k = _bf16((slots.numel(), hkv, dim), generator, gpu_device)
    rows_v = _bf16((slots.numel(), hkv, dim), generator, gpu_device)
    key_pool[slots] = rows_k
    value_pool[slots] = rows_v
    spans = [(slots, 1200, 1232), (slots, 2900, 2916), (slots, 2990, 3000)]
    report(f"pool of {pool} slots ({pool * hkv * dim * 2 / 2**30:.2f} GiB per buffer), top slot {int(slots.max())}")
    plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim, pool_size=pool)
    query = _bf16((plan.num_queries, hq, dim), generator, gpu_device)
    got = plan.run(query, key_pool, value_pool)
    # The same rows at slots 0 .. 2,999 of a small pool.
    small = torch.arange(slots.numel(), device=gpu_device)
    small_spans = [(small, start, end) for _, start, end in spans]
    small_plan = RepairAttentionPlan(small_spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim,
                                     pool_size=slots.numel())
    want = small_plan.run(query, rows_k, rows_v)
    torch.cuda.synchronize(gpu_device)
    assert torch.equal(got, want)
    del key_pool, value_pool
    _check(small_spans, query, rows_k, rows_v, want, 1.0 / math.sqrt(dim))


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_full_size_workload_sampled(gpu_device, name):
    """The benchmark workloads at full size with the plan's own chunks (c5:
    511 spans over a 32,768-token request, whole key ranges of up to 32,768
    keys (four slot-list refills), no combine; c3: 448 eight-query spans of 64
    requests sharing tiles, 6,208-key chunks and their combine): the last row
    of every span (the one that sees the most keys) and
    64 random rows, each checked against fp32 torch attention on the device,
    within the same bound."""

    from legolink_amd.link_plan import contiguous_ranges
    from legolink_amd.workloads import make_workload

    workload = make_workload(name)
    shape = workload.shape
    hq = 28
    generator = torch.Generator(device=gpu_device).manual_seed(7)
    key_pool = _bf16((workload.num_slots, shape.kv_heads, shape.head_dim), generator, gpu_device)
    value_pool = _bf16((workload.num_slots, shape.kv_heads, shape.head_dim), generator, gpu_device)
    spans = []
    for destination, plan in workload.link_requests()[1]:
        slots = torch.from_numpy(destination).to(gpu_device)
        spans += [(slots, int(s), int(e)) for s, e in contiguous_ranges(plan["imp_indices"])]
    plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=shape.kv_heads, head_dim=shape.head_dim,
                               pool_size=workload.num_slots)
    report(f"{name}: {len(spans)} spans, {plan.num_queries} queries, plan {plan.info}")
    query = _bf16((plan.num_queries, hq, shape.head_dim), generator, gpu_device)
    scale = 1.0 / math.sqrt(shape.head_dim)
    got = plan.run(query, key_pool, value_pool, scale=scale).float()
    torch.cuda.synchronize(gpu_device)
    rng = np.random.default_rng(3)
    starts = np.cumsum([0] + [e - s for _, s, e in spans])
    group = hq // shape.kv_heads
    worst = 0.0
    rows = [(index, end - start - 1) for index, (_, start, end) in enumerate(spans)]
    for index in rng.choice(len(spans), size=64, replace=True):
        _, start, end = spans[index]
        rows.append((int(index), int(rng.integers(0, end - start))))
    for index, row in rows:
        slots, start, end = spans[index]
        q = query[starts[index] + row].float()                                  # [hq, d]
        keys = key_pool[slots[: start + row + 1]].float()                       # [n, hkv, d]
        values = value_pool[slots[: start + row + 1]].float()
        keys = keys.repeat_interleave(group, dim=1).permute(1, 0, 2)            # [hq, n, d]
        values = values.repeat_interleave(group, dim=1).permute(1, 0, 2)
        weights = torch.softmax((keys @ q[:, :, None])[:, :, 0] * scale, dim=-1)  # [hq, n]
        want = (weights[:, None, :] @ values)[:, 0, :]
        magnitude = (weights[:, None, :] @ values.abs())[:, 0, :]
        bound = 2.0 ** -7 * (magnitude + want.abs()) + 1e-5
        err = (got[starts[index] + row] - want).abs()
        worst = max(worst, float((err / bound).max()))
        assert bool((err <= bound).all()), f"span {index} row {row}: max err {float(err.max()):.3g}"
    report(f"{len(rows)} rows checked; largest error / bound vs fp32: {worst:.3f}")


def test_span_checks_follow_the_reference(gpu_device):
    slots = torch.arange(10, device=gpu_device)
    for bad, message in [((slots.view(2, 5), 1, 3), "rank 1"), ((slots, 3, 3), "invalid repair range"),
                         ((slots, 5, 12), "shorter than repair_end")]:
        with pytest.raises(SparseRepairAttentionError, match=message):
            RepairAttentionPlan([bad], num_q_heads=4, num_kv_heads=2, head_dim=64)
