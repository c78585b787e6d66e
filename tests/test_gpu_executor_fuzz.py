"""Seeded random plans through the whole executor, against the oracle.

Each case registers random blocks (consecutive, offset or explicit compile
positions; some captured into the snapshot arena), derives a plan with a
random fresh prefix, gaps between blocks, recompute counts and mutable
suffix (resolve_link_plan), and links it with a random fused mode, repair
awareness and repair-row form, then writes the repaired rows back.  The
expected pools come from the maps oracle (plan-order maps of the reference's
map construction) and the pool oracle, per source (pool or arena), in the
rounding the fused mode selects.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from legolink_amd.link_plan import resolve_link_plan
from legolink_amd.link_runtime import KVLinkExecutor, KVPool, SnapshotArena
from legolink_amd.registry import LegoLinkBlockRegistry
from legolink_amd.rope import RotarySpec
from oracle import kv_link_oracle as ko
from oracle import link_maps_oracle as lmo
from tests.gpu_helpers import bits, report

pytestmark = pytest.mark.gpu


def _pool(layers, slots, heads, dim, device, generator):
    def layer():
        return torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=device, generator=generator)

    return KVPool([layer() for _ in range(layers)], [layer() for _ in range(layers)])


@pytest.mark.parametrize("seed", range(128))
def test_random_plan_through_the_executor_matches_oracle(gpu_device, seed):
    rng = np.random.default_rng([7, seed])
    layers = int(rng.choice([1, 3, 28]))
    heads = int(rng.choice([1, 4]))
    dim = int(rng.choice([64, 128]))
    slots = 8192
    generator = torch.Generator(device=gpu_device).manual_seed(seed)
    pool = _pool(layers, slots, heads, dim, gpu_device, generator)
    arena = SnapshotArena.allocate(num_slots=2048, num_layers=layers, num_heads=heads, head_dim=dim,
                                   device=gpu_device)
    perm = rng.permutation(slots)
    cursor = 0
    registry = LegoLinkBlockRegistry()
    executor_modes = ["disabled", "auto", "required"]
    n_blocks = int(rng.integers(1, 7))
    blocks = {}
    for index in range(n_blocks):
        length = int(rng.integers(1, 300))
        kind = int(rng.integers(4))
        if kind == 0:
            positions = None
        elif kind == 1:
            positions = (np.arange(length) + int(rng.integers(1, 600))).tolist()
        else:  # explicit, increasing with holes
            positions = np.cumsum(rng.integers(1, 3, size=length)).tolist()
        tokens = rng.integers(0, 50_000, size=length).tolist()
        source = perm[cursor:cursor + length]
        cursor += length
        blocks[f"b{index}"] = {"tokens": tokens, "source": source, "positions": positions,
                               "clone": bool(rng.random() < 0.2)}
    order = [f"b{i}" for i in rng.permutation(n_blocks)]
    prefix_tokens = int(rng.integers(0, 30))
    gaps = [int(rng.integers(0, 4)) if rng.random() < 0.3 else 0 for _ in range(n_blocks - 1)]
    plan = {"cache_keys": order, "recompute_initial_tokens": int(rng.integers(0, 20))}
    host = rng.integers(0, 50_000, size=prefix_tokens + sum(gaps) + int(rng.integers(1, 20))).tolist()
    if prefix_tokens or any(gaps):
        plan["physical_prefix_token_count"] = prefix_tokens
        plan["physical_interblock_fresh_token_counts"] = gaps
    has_clone = any(block["clone"] for block in blocks.values())
    fused_mode = executor_modes[int(rng.integers(2 if has_clone else 3))]
    boundary_repair_aware = bool(rng.random() < 0.7)
    compact = bool(rng.random() < 0.5)
    report(f"executor fuzz {seed}: layers={layers} heads={heads} dim={dim} blocks={n_blocks} "
           f"clone={[blocks[k]['clone'] for k in order]} prefix={prefix_tokens} gaps={gaps} "
           f"mode={fused_mode} aware={boundary_repair_aware} compact={compact}")

    executor = KVLinkExecutor(registry, RotarySpec.for_theta(2048, dim), end_layer=layers, arena=arena,
                              fused_mode=fused_mode)
    executor.capture_blocks(pool, [
        {"cache_key": key, "token_ids": block["tokens"],
         "slots": torch.from_numpy(block["source"]).to(gpu_device),
         "storage_mode": "clone" if block["clone"] else "reference",
         "compile_local_positions": block["positions"]}
        for key, block in blocks.items()])
    linked = resolve_link_plan(registry.get_legolink_block_tokens, host, plan)
    destination = perm[cursor:cursor + len(linked)]
    before_k = [bits(k) for k in pool.k_buffer]
    before_v = [bits(v) for v in pool.v_buffer]
    arena_k = [bits(k) for k in arena.k_buffer]
    arena_v = [bits(v) for v in arena.v_buffer]

    prepared = executor.prepare_link(pool, torch.from_numpy(destination).to(gpu_device), plan,
                                     boundary_repair_aware=boundary_repair_aware, compact_repair_rows=compact)
    prepared.launch()
    rows = int(prepared.repair_offsets.size)
    repaired_k = torch.randn(layers, rows, heads, dim, generator=generator, device=gpu_device).to(torch.bfloat16)
    repaired_v = torch.randn_like(repaired_k)
    if rows:
        prepared.write_repaired(repaired_k, repaired_v)
    torch.cuda.synchronize(gpu_device)
    executor.check_skipped_rows()

    # Expected: the oracle's maps of the plan, then the link per source.
    oracle_blocks = []
    for entry, key in zip(plan["block_ranges"], order):
        handle = registry.lookup_legolink_blocks([key]).matched_handles[0]
        oracle_blocks.append({"start": int(entry["start_token"]),
                              "source_slots": handle.kv_slots.cpu().numpy(),
                              "local_positions": np.asarray(handle.compile_local_positions, dtype=np.int64),
                              "set": 1 if blocks[key]["clone"] else 0})
    imp = plan["imp_indices"] if boundary_repair_aware else []
    maps = lmo.concatenated_maps(oracle_blocks, destination, imp)
    assert rows == maps["repair_offsets"].size
    rounding = ko.EAGER if prepared.rounding == "eager" else ko.FUSED
    assert prepared.rounding == ("eager" if fused_mode == "disabled" or has_clone else "fused")
    repair_mask = np.zeros(maps["source_slots"].size, dtype=np.uint8)
    repair_mask[maps["repair_offsets"]] = 1
    table = executor.rotary_by_layer[0].cos_sin_cache.cpu().numpy()
    want_k, want_v = before_k, before_v
    first_set = oracle_blocks[0]["set"]
    for source_set, (src_k, src_v) in ((0, (before_k, before_v)), (1, (arena_k, arena_v))):
        pick = maps["sets"] == source_set
        if not pick.any():
            continue
        # The identity prefix is the first block's tokens: the first ones of its set.
        prefix = maps["prefix_token_count"] if source_set == first_set else 0
        want_k, want_v = ko.link_pool(
            want_k, want_v, maps["source_slots"][pick], maps["destination_slots"][pick],
            maps["local_positions"][pick], maps["global_positions"][pick], table, key_dtype=ko.BF16,
            cache_dtype=ko.F32, rotary_dim=dim, neox=True, prefix=prefix, repair_mask=repair_mask[pick],
            source_key_layers=src_k, source_value_layers=src_v, rounding=rounding)
    if rows:
        want_k, want_v = ko.scatter_rows(want_k, want_v, maps["destination_slots"][maps["repair_offsets"]],
                                         bits(repaired_k), bits(repaired_v))
    for layer in range(layers):
        assert np.array_equal(bits(pool.k_buffer[layer]), want_k[layer]), f"seed {seed}: K layer {layer}"
        assert np.array_equal(bits(pool.v_buffer[layer]), want_v[layer]), f"seed {seed}: V layer {layer}"


@pytest.mark.parametrize("seed", range(48))
def test_random_batches_through_the_executor_match_oracle(gpu_device, seed):
    """prepare_links over 2-4 requests drawn from shared registered blocks (in
    any order, some clone blocks), with repair rows: every request's rows
    equal the oracle's, and the write-back covers the requests' repair rows
    request after request."""

    rng = np.random.default_rng([11, seed])
    layers, heads, dim, slots = int(rng.choice([1, 3, 28])), 4, 128, 16384
    generator = torch.Generator(device=gpu_device).manual_seed(seed)
    pool = _pool(layers, slots, heads, dim, gpu_device, generator)
    arena = SnapshotArena.allocate(num_slots=4096, num_layers=layers, num_heads=heads, head_dim=dim,
                                   device=gpu_device)
    perm = rng.permutation(slots)
    cursor = 0
    registry = LegoLinkBlockRegistry()
    catalogue = {}
    for index in range(int(rng.integers(2, 8))):
        length = int(rng.integers(1, 200))
        catalogue[f"c{index}"] = {"tokens": rng.integers(0, 50_000, size=length).tolist(),
                                  "source": perm[cursor:cursor + length], "clone": bool(rng.random() < 0.2),
                                  "positions": None if rng.random() < 0.7 else
                                  (np.arange(length) + int(rng.integers(1, 300))).tolist()}
        cursor += length
    has_clone = any(block["clone"] for block in catalogue.values())
    fused_mode = ["disabled", "auto", "required"][int(rng.integers(2 if has_clone else 3))]
    executor = KVLinkExecutor(registry, RotarySpec.for_theta(4096, dim), end_layer=layers, arena=arena,
                              fused_mode=fused_mode)
    executor.capture_blocks(pool, [
        {"cache_key": key, "token_ids": block["tokens"],
         "slots": torch.from_numpy(block["source"]).to(gpu_device),
         "storage_mode": "clone" if block["clone"] else "reference",
         "compile_local_positions": block["positions"]}
        for key, block in catalogue.items()])
    keys = list(catalogue)
    requests = []
    for _ in range(int(rng.integers(2, 5))):
        order = [keys[i] for i in rng.choice(len(keys), size=int(rng.integers(1, len(keys) + 1)), replace=False)]
        plan = {"cache_keys": order, "recompute_initial_tokens": int(rng.integers(0, 12))}
        linked = resolve_link_plan(registry.get_legolink_block_tokens,
                                   rng.integers(0, 50_000, size=int(rng.integers(1, 10))).tolist(), plan)
        destination = perm[cursor:cursor + len(linked)]
        cursor += len(linked)
        requests.append((destination, plan, order))
    report(f"executor batch fuzz {seed}: layers={layers} requests={[r[2] for r in requests]} "
           f"clone={[catalogue[k]['clone'] for k in keys]} mode={fused_mode}")
    before_k = [bits(k) for k in pool.k_buffer]
    before_v = [bits(v) for v in pool.v_buffer]
    arena_k = [bits(k) for k in arena.k_buffer]
    arena_v = [bits(v) for v in arena.v_buffer]
    prepared = executor.prepare_links(pool, [(torch.from_numpy(d).to(gpu_device), p) for d, p, _ in requests],
                                      boundary_repair_aware=True, compact_repair_rows=bool(seed % 2))
    prepared.launch()
    rows = int(prepared.repair_offsets.size)
    repaired_k = torch.randn(layers, rows, heads, dim, generator=generator, device=gpu_device).to(torch.bfloat16)
    repaired_v = torch.randn_like(repaired_k)
    if rows:
        prepared.write_repaired(repaired_k, repaired_v)
    torch.cuda.synchronize(gpu_device)
    executor.check_skipped_rows()

    # Rounding per request, as each request's own link decides it.
    holds_clone = [any(catalogue[key]["clone"] for key in order) for _, _, order in requests]
    request_roundings = ["eager" if fused_mode == "disabled" or clone else "fused" for clone in holds_clone]
    assert prepared.request_roundings == request_roundings
    table = executor.rotary_by_layer[0].cos_sin_cache.cpu().numpy()
    want_k, want_v = before_k, before_v
    repair_destinations = []
    for (destination, plan, order), request_rounding in zip(requests, request_roundings):
        rounding = ko.EAGER if request_rounding == "eager" else ko.FUSED
        blocks = []
        for entry, key in zip(plan["block_ranges"], order):
            handle = registry.lookup_legolink_blocks([key]).matched_handles[0]
            blocks.append({"start": int(entry["start_token"]), "source_slots": handle.kv_slots.cpu().numpy(),
                           "local_positions": np.asarray(handle.compile_local_positions, dtype=np.int64),
                           "set": 1 if catalogue[key]["clone"] else 0})
        maps = lmo.concatenated_maps(blocks, destination, plan["imp_indices"])
        repair_destinations.append(maps["destination_slots"][maps["repair_offsets"]])
        mask = np.zeros(maps["source_slots"].size, dtype=np.uint8)
        mask[maps["repair_offsets"]] = 1
        for source_set, (src_k, src_v) in ((0, (before_k, before_v)), (1, (arena_k, arena_v))):
            pick = maps["sets"] == source_set
            if pick.any():
                prefix = maps["prefix_token_count"] if source_set == blocks[0]["set"] else 0
                want_k, want_v = ko.link_pool(
                    want_k, want_v, maps["source_slots"][pick], maps["destination_slots"][pick],
                    maps["local_positions"][pick], maps["global_positions"][pick], table, key_dtype=ko.BF16,
                    cache_dtype=ko.F32, rotary_dim=dim, neox=True, prefix=prefix, repair_mask=mask[pick],
                    source_key_layers=src_k, source_value_layers=src_v, rounding=rounding)
    repair_destinations = np.concatenate(repair_destinations)
    assert rows == repair_destinations.size
    if rows:
        want_k, want_v = ko.scatter_rows(want_k, want_v, repair_destinations, bits(repaired_k), bits(repaired_v))
    for layer in range(layers):
        assert np.array_equal(bits(pool.k_buffer[layer]), want_k[layer]), f"seed {seed}: K layer {layer}"
        assert np.array_equal(bits(pool.v_buffer[layer]), want_v[layer]), f"seed {seed}: V layer {layer}"
