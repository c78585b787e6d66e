"""The link and the repair pass together, on the HIP path, at the Qwen2.5-7B
shape: the reference's end-to-end check (tests/pic/test_pic_end_to_end_small.py:14-91)
on c2's block geometry.

That test compiles blocks with RoPE at their local positions, links them into
a request, runs the repair attention over the linked physical slots, writes
the repaired rows, and checks that the attention equals causal attention over
keys rotated directly to their global positions.  Here:

* every token's raw key is rotated (fp64, textbook RoPE) to its block's
  compile-time position and stored in bf16 at its source slot;
* the executor links c2's 16 blocks (32,768 tokens, 15 seams of 16
  imp_indices) into the request's slots, repair rows left out;
* per layer, that layer's repaired rows are written first (a one-layer
  ll_kv_scatter_rows, the repair pass's set_kv_buffer,
  flashinfer_sparse_repair.py:2235-2239), then the HIP repair attention runs
  with 28 query heads over the 4 KV heads.

Checks, per layer and output element (size = the attention of |V|, as in the
attention tests):

A. against the fp64 attention oracle over the linked pool as read back:
   |got - pool| <= 2^-7 (size + |pool|) + 1e-5 (the kernel's own bound);
B. the linked pool against keys rotated directly to their global positions:
   with d_j = scale * q . (K_linked[j] - K_direct[j]) over the query's visible
   keys, the softmax weights move by at most a factor e^(max d - min d), so
   |pool - direct| <= (e^(max d - min d) - 1) * size;
C. end to end, |got - direct| <= bound A + bound B;
D. the repaired rows were written before the attention read them: the output
   is off the attention over the pool as it was before the write.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from legolink_amd import kv_link
from legolink_amd.link_plan import contiguous_ranges
from legolink_amd.link_runtime import KVLinkExecutor, KVPool
from legolink_amd.registry import LegoLinkBlockRegistry
from legolink_amd.repair_attention import RepairAttentionPlan
from legolink_amd.rope import RotarySpec, build_cos_sin_cache
from legolink_amd.workloads import make_workload
from oracle import attention_oracle as ao
from oracle import kv_link_oracle as ko
from tests import rope_math
from tests.gpu_helpers import bits, report

pytestmark = pytest.mark.gpu


def _to_bf16(values: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(ko.f32_to_bf16_bits(values.astype(np.float32)).view(np.int16)).view(torch.bfloat16).to(device)


def _f64(tensor: torch.Tensor) -> np.ndarray:
    return tensor.float().cpu().numpy().astype(np.float64)


def _attention_with_shift(query, key_pool, key_direct, values, start, end, scale):
    """fp64 attention of one span over the pool's keys, over the direct keys,
    the size (|V|), and per query and head the spread of d_j (max - min)."""

    q_pos = np.arange(start, end)
    visible = ao.logical_causal_mask(q_pos, np.arange(end))
    pool = ao.gqa_attention(query, key_pool, values, visible, scale=scale)
    direct = ao.gqa_attention(query, key_direct, values, visible, scale=scale)
    size = ao.gqa_attention(query, key_pool, np.abs(values), visible, scale=scale)
    hq, hkv = query.shape[1], key_pool.shape[1]
    group = hq // hkv
    spread = np.zeros((end - start, hq))
    diff = key_pool - key_direct
    for h in range(hq):
        shift = (query[:, h, :] @ diff[:, h // group, :].T) * scale       # [q, kv]
        shift = np.where(visible, shift, np.nan)
        spread[:, h] = np.nanmax(shift, axis=1) - np.nanmin(shift, axis=1)
    return pool, direct, size, spread


def test_link_then_repair_attention_equals_direct_rotation_c2(gpu_device):
    workload = make_workload("c2")
    shape = workload.shape
    layers, hq, hkv, dim = 2, 28, shape.kv_heads, shape.head_dim
    assert (hkv, dim) == (4, 128)
    rng = np.random.default_rng(20260824)
    blocks, requests = workload.link_requests()
    (request_slots, plan), = requests
    tokens = int(request_slots.size)
    report(f"composition: {len(blocks)} blocks, {tokens} tokens, {len(plan['imp_indices'])} imp_indices, "
           f"{layers} layers, {hq}/{hkv} heads")

    # Raw keys and values by request position; blocks compiled at their local
    # positions and stored at their source slots.
    raw_k = rng.standard_normal((layers, tokens, hkv, dim))
    raw_v = rng.standard_normal((layers, tokens, hkv, dim))
    generator = torch.Generator(device=gpu_device).manual_seed(5)
    keys = [torch.randn(workload.num_slots, hkv, dim, generator=generator, device=gpu_device).to(torch.bfloat16)
            for _ in range(layers)]
    values = [torch.randn(workload.num_slots, hkv, dim, generator=generator, device=gpu_device).to(torch.bfloat16)
              for _ in range(layers)]
    registry = LegoLinkBlockRegistry()
    for key, (source, local) in blocks.items():
        entry = plan["block_ranges"][plan["cache_keys"].index(key)]
        positions = np.arange(entry["start_token"], entry["end_token"])
        for layer in range(layers):
            compiled = rope_math.rotate(raw_k[layer, positions], local, dim, theta=workload.theta)
            slots = torch.from_numpy(source).to(gpu_device)
            keys[layer][slots] = _to_bf16(compiled, gpu_device)
            values[layer][slots] = _to_bf16(raw_v[layer, positions], gpu_device)
        registry.register_legolink_block(key, range(source.size), torch.from_numpy(source).to(gpu_device),
                                         compile_local_positions=local.tolist())
    table = build_cos_sin_cache(workload.max_position + 1, dim, theta=workload.theta).to(gpu_device)
    executor = KVLinkExecutor(registry, RotarySpec(table, rotary_dim=dim), end_layer=layers, fused_mode="required")
    pool = KVPool(keys, values)
    destination = torch.from_numpy(request_slots).to(gpu_device)
    prepared = executor.prepare_link(pool, destination, plan, boundary_repair_aware=True, compact_repair_rows=True)
    prepared.launch()
    executor.check_skipped_rows()

    repair_positions = np.asarray(plan["imp_indices"], dtype=np.int64)
    repair_slots = prepared.repair_destination_slots
    assert np.array_equal(repair_slots.cpu().numpy(), request_slots[repair_positions])
    spans = [(destination, int(s), int(e)) for s, e in contiguous_ranges(plan["imp_indices"])]
    attention = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim,
                                    pool_size=workload.num_slots)
    scale = 1.0 / math.sqrt(dim)
    worst = {"A": 0.0, "B": 0.0, "C": 0.0}
    off_before = 0.0
    for layer in range(layers):
        # The repaired rows differ strongly from what the slots held before.
        repaired_k = (3.0 * torch.randn(1, len(repair_positions), hkv, dim, generator=generator,
                                        device=gpu_device)).to(torch.bfloat16)
        repaired_v = (4.0 * torch.randn(1, len(repair_positions), hkv, dim, generator=generator,
                                        device=gpu_device)).to(torch.bfloat16)
        query = torch.randn(attention.num_queries, hq, dim, generator=generator, device=gpu_device).to(torch.bfloat16)
        before_k = _f64(keys[layer][destination])
        before_v = _f64(values[layer][destination])
        # Layer l: write its repaired rows, then attend.
        kv_link.scatter_kv_rows_inplace(key_buffers=[keys[layer]], value_buffers=[values[layer]],
                                        destination_slots=repair_slots, repaired_keys=repaired_k,
                                        repaired_values=repaired_v)
        got = _f64(attention.run(query, keys[layer], values[layer], scale=scale))
        torch.cuda.synchronize(gpu_device)
        report(f"composition layer {layer}: kernels done, checking {len(spans)} spans")

        linked_k = _f64(keys[layer][destination])          # by request position
        linked_v = _f64(values[layer][destination])
        direct_k = rope_math.rotate(raw_k[layer], np.arange(tokens), dim, theta=workload.theta)
        direct_k[repair_positions] = _f64(repaired_k[0])
        # V is a bit copy of the bf16 source rows; the repaired rows replace theirs.
        assert np.array_equal(bits(values[layer][destination])[~np.isin(np.arange(tokens), repair_positions)],
                              ko.f32_to_bf16_bits(raw_v[layer].astype(np.float32))[
                                  ~np.isin(np.arange(tokens), repair_positions)])
        before_k_all = before_k.copy()
        before_v_all = before_v.copy()
        q_all = _f64(query)
        cursor = 0
        for _, start, end in spans:
            n = end - start
            q = q_all[cursor : cursor + n]
            part = got[cursor : cursor + n]
            pool_out, direct_out, size, spread = _attention_with_shift(
                q, linked_k[:end], direct_k[:end], linked_v[:end], start, end, scale)
            bound_a = 2.0 ** -7 * (size + np.abs(pool_out)) + 1e-5
            bound_b = np.expm1(spread)[:, :, None] * size + 1e-12
            err_a = np.abs(part - pool_out)
            err_b = np.abs(pool_out - direct_out)
            err_c = np.abs(part - direct_out)
            assert (err_a <= bound_a).all(), f"layer {layer} span [{start}, {end}): kernel vs linked-pool oracle"
            assert (err_b <= bound_b).all(), f"layer {layer} span [{start}, {end}): linked pool vs direct rotation"
            assert (err_c <= bound_a + bound_b).all(), f"layer {layer} span [{start}, {end}): end to end"
            worst["A"] = max(worst["A"], float((err_a / bound_a).max()))
            worst["B"] = max(worst["B"], float((err_b / bound_b).max()))
            worst["C"] = max(worst["C"], float((err_c / (bound_a + bound_b)).max()))
            # The same span over the rows as they were before the write-back.
            visible = ao.logical_causal_mask(np.arange(start, end), np.arange(end))
            stale = ao.gqa_attention(q, before_k_all[:end], before_v_all[:end], visible, scale=scale)
            off_before = max(off_before, float((np.abs(part - stale) / bound_a).max()))
            assert float(spread.max()) < 0.1  # the linked keys are the directly rotated ones, closely
            cursor += n
        assert cursor == attention.num_queries
    report(f"composition: largest error / bound A {worst['A']:.3f}, B {worst['B']:.3f}, C {worst['C']:.3f}; "
           f"attention over the rows before the write-back is off by {off_before:.1f}x the bound")
    assert off_before > 10.0
