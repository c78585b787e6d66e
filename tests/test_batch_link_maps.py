"""The batched map builder (``KVLinkExecutor.build_batch_link_maps``) against
the per-request builder it replaces in ``prepare_links``: the same LinkMaps
field by field on random batches, and the same error where a request's own
link fails (pic_runtime.py:4905-5013 raises per block).  CPU tensors only:
the builder reads registry records and plan ranges, not device memory."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from legolink_amd.errors import LinkRuntimeError
from legolink_amd.link_runtime import KVLinkExecutor, LinkMaps
from legolink_amd.registry import LegoLinkBlockRegistry
from legolink_amd.rope import RotarySpec, build_cos_sin_cache

CPU = torch.device("cpu")


def _registry(rng, count=12):
    registry = LegoLinkBlockRegistry()
    lengths = {}
    for index in range(count):
        length = int(rng.integers(1, 40))
        kind = index % 3
        if kind == 0:  # compiled at 0..n-1
            local = None
        elif kind == 1:  # compiled behind a prefix
            local = list(range(7, 7 + length))
        else:  # not consecutive
            local = sorted(rng.choice(200, size=length, replace=False).tolist())
        registry.register_legolink_block(f"b{index}", range(length),
                                         torch.from_numpy(rng.choice(4096, size=length, replace=False)),
                                         compile_local_positions=local,
                                         storage_mode="clone" if index % 5 == 4 else "reference")
        lengths[f"b{index}"] = length
    return registry, lengths


def _request(rng, lengths, *, dtype=torch.int64, repair_as=list):
    keys = [str(k) for k in rng.choice(sorted(lengths), size=int(rng.integers(1, 6)))]
    ranges, start = [], 0
    for key in keys:
        ranges.append({"start_token": start, "end_token": start + lengths[key]})
        start += lengths[key]
    total = start + int(rng.integers(0, 5))
    imp = rng.integers(-3, total + 3, size=int(rng.integers(0, 9))).tolist()
    plan = {"cache_keys": keys, "block_ranges": ranges, "imp_indices": repair_as(imp)}
    return torch.from_numpy(rng.choice(1 << 20, size=total, replace=False)).to(dtype), plan


def _executor(registry):
    return KVLinkExecutor(registry, RotarySpec(build_cos_sin_cache(64, 128, theta=1e6), rotary_dim=128),
                          end_layer=1)


def _assert_same(a: LinkMaps, b: LinkMaps):
    for name in ("starts", "counts", "source_ptrs", "local_ptrs", "local_starts", "sets", "destination_bases"):
        x, y = getattr(a.blocks, name), getattr(b.blocks, name)
        if x is None or y is None:  # destination bases of a single request
            assert x is None and y is None, name
            continue
        assert x.dtype == y.dtype and np.array_equal(x, y), name
    assert a.request_slots.dtype == b.request_slots.dtype == torch.int64
    assert torch.equal(a.request_slots, b.request_slots)
    assert a.repair_positions.dtype == b.repair_positions.dtype
    assert np.array_equal(a.repair_positions, b.repair_positions)
    assert np.array_equal(a.leading_blocks, b.leading_blocks)
    assert (a.prefix_token_count, a.max_position, a.request_count) == (b.prefix_token_count, b.max_position,
                                                                        b.request_count)
    assert len(a.handles) == len(b.handles) and all(h is g for h, g in zip(a.handles, b.handles))
    assert np.array_equal(a.block_requests, b.block_requests)
    assert np.array_equal(a.request_has_clone(), b.request_has_clone())


@pytest.mark.parametrize("seed", range(12))
def test_batched_maps_equal_the_per_request_maps(seed):
    rng = np.random.default_rng(seed)
    registry, lengths = _registry(rng)
    executor = _executor(registry)
    kinds = [(torch.int64, list), (torch.int32, list), (torch.int64, np.asarray),
             (torch.int32, lambda v: torch.tensor(v, dtype=torch.int64))]
    requests = [_request(rng, lengths, dtype=kinds[i % 4][0], repair_as=kinds[i % 4][1])
                for i in range(int(rng.integers(2, 9)))]
    batched = executor.build_batch_link_maps(requests, device=CPU)
    one_by_one = LinkMaps.batch([executor.build_link_maps(s, p, device=CPU) for s, p in requests])
    _assert_same(batched, one_by_one)
    # Identity first blocks were found: a block compiled at 0..n-1 placed first.
    assert batched.leading_blocks.sum() == sum(
        1 for _, plan in requests if int(plan["cache_keys"][0][1:]) % 3 == 0)


def test_batched_maps_of_one_request_are_its_maps():
    rng = np.random.default_rng(99)
    registry, lengths = _registry(rng)
    executor = _executor(registry)
    slots, plan = _request(rng, lengths)
    _assert_same(executor.build_batch_link_maps([(slots, plan)], device=CPU),
                 executor.build_link_maps(slots, plan, device=CPU))
    with pytest.raises(LinkRuntimeError, match="no requests"):
        executor.build_batch_link_maps([], device=CPU)


def _faults():
    def missing(plan):
        plan["cache_keys"][-1] = "absent"

    def count(plan):
        plan["block_ranges"][-1]["end_token"] += 1

    def outside(plan):
        for r in plan["block_ranges"]:
            r["start_token"] += 10_000
            r["end_token"] += 10_000

    def negative(plan):
        for r in plan["block_ranges"]:
            r["start_token"] -= 50
            r["end_token"] -= 50

    def lengths(plan):
        plan["cache_keys"] = plan["cache_keys"] + ["b0"]

    def empty(plan):
        plan["cache_keys"], plan["block_ranges"] = [], []

    def no_ranges(plan):
        del plan["block_ranges"]

    return [missing, count, outside, negative, lengths, empty, no_ranges]


@pytest.mark.parametrize("fault", _faults(), ids=lambda f: f.__name__)
def test_a_faulty_request_raises_what_its_own_link_raises(fault):
    rng = np.random.default_rng(5)
    registry, lengths = _registry(rng)
    executor = _executor(registry)
    requests = [_request(rng, lengths) for _ in range(4)]
    fault(requests[2][1])
    with pytest.raises(LinkRuntimeError) as own:
        executor.build_link_maps(*requests[2], device=CPU)
    with pytest.raises(LinkRuntimeError) as batched:
        executor.build_batch_link_maps(requests, device=CPU)
    assert str(batched.value) == str(own.value)


def test_a_stale_block_fails_the_batch():
    rng = np.random.default_rng(6)
    registry, lengths = _registry(rng)
    executor = _executor(registry)
    requests = [_request(rng, lengths) for _ in range(3)]
    stale = requests[1][1]["cache_keys"][0]
    registry.evict_legolink_block(stale)
    with pytest.raises(LinkRuntimeError, match=stale):
        executor.build_batch_link_maps(requests, device=CPU)


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("compact", [True, False])
def test_entry_flags_follow_each_entrys_request(seed, compact):
    """set_entry_flags spreads a per-run flag (here: the run's request holds a
    clone block) over a set's map entries; checked against the entries'
    requests rebuilt token by token from the plan's own runs."""

    from legolink_amd import link_maps

    rng = np.random.default_rng([5, seed])
    registry, lengths = _registry(rng)
    executor = _executor(registry)
    requests = [_request(rng, lengths) for _ in range(int(rng.integers(2, 6)))]
    maps = executor.build_batch_link_maps(requests, device=CPU)
    clone = maps.request_has_clone()
    for request in range(maps.request_count):
        own = maps.blocks.sets[maps.block_requests == request]
        assert bool(clone[request]) == bool((own == 1).any())
    plan = link_maps.plan_segments(maps.blocks, maps.repair_positions, compact=compact,
                                   leading_blocks=maps.leading_blocks)
    run_request = maps.block_requests[plan.segment_blocks]
    table = plan.table
    field = link_maps._FIELD
    for source_set in (0, 1):
        flags = link_maps.set_entry_flags(plan, source_set, clone[run_request], compact=compact)
        want = np.full(plan.map_counts[source_set], 255, dtype=np.int64)
        entries = plan.run_entries(compact)
        for run in np.flatnonzero(table[:, field["map_set"]] == source_set):
            offset = table[run, field["map_offset"]]
            assert (want[offset:offset + entries[run]] == 255).all()  # runs do not overlap
            want[offset:offset + entries[run]] = clone[run_request[run]]
        assert (want != 255).all()
        assert np.array_equal(flags, want.astype(np.uint8))
