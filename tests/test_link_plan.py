"""Plan derivation, registry and executor map building against the reference's
known answers (no GPU)."""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from legolink_amd.errors import LinkRuntimeError
from legolink_amd.link_plan import ResolvedLinkPlan, contiguous_ranges, resolve_link_plan
from legolink_amd.link_runtime import KVLinkExecutor, KVPool
from legolink_amd.registry import LegoLinkBlockRegistry
from legolink_amd.rope import RotarySpec

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def test_contiguous_ranges_known_answer():
    case = GOLDEN["contiguous_ranges"]
    assert contiguous_ranges(case["input"]) == [tuple(r) for r in case["expected"]]
    for rejected in case["rejected"]:
        with pytest.raises(LinkRuntimeError, match="strictly increasing"):
            contiguous_ranges(rejected)
    assert contiguous_ranges([]) == []


@pytest.mark.parametrize("case", GOLDEN["plan_derivation"]["cases"], ids=lambda c: c["name"])
def test_plan_derivation_known_answers(case):
    plan = {"cache_keys": list(case["cache_keys"]), **{k: v for k, v in case["link_plan"].items() if k != "normalized_layout"}}
    if "block_ids" in case:
        plan["block_ids"] = list(case["block_ids"])
    linked = resolve_link_plan(case["blocks"], case["mutable_input_ids"], plan)
    assert plan["imp_indices"] == case["expected_imp_indices"]
    assert plan["kvlink"] == plan["imp_indices"]
    if "expected_linked" in case:
        assert linked == case["expected_linked"]
    if "expected_mutable_start_token" in case:
        assert plan["mutable_start_token"] == case["expected_mutable_start_token"]
    if "expected_block_ranges" in case:
        assert plan["block_ranges"] == case["expected_block_ranges"]
    if "expected_block_starts" in case:
        assert [r["start_token"] for r in plan["block_ranges"]] == case["expected_block_starts"]
    assert plan["total_token_count"] == len(linked)


def test_plan_is_deterministic_and_frozen():
    blocks = {"a": [1, 2, 3], "b": [4, 5]}
    plan_one = {"cache_keys": ["a", "b"], "recompute_initial_tokens": 1}
    plan_two = dict(plan_one)
    resolve_link_plan(blocks, [9], plan_one)
    resolve_link_plan(lambda key: blocks.get(key), [9], plan_two)
    assert plan_one == plan_two
    frozen = ResolvedLinkPlan.freeze_ranges(plan_one["block_ranges"])
    assert hash(frozen) == hash(ResolvedLinkPlan.freeze_ranges(plan_two["block_ranges"]))


def test_plan_errors_follow_the_reference_messages():
    with pytest.raises(LinkRuntimeError, match="cache_keys must be non-empty"):
        resolve_link_plan({}, [1], {"cache_keys": []})
    with pytest.raises(LinkRuntimeError, match="not compiled in this scheduler: x"):
        resolve_link_plan({}, [1], {"cache_keys": ["x"]})
    with pytest.raises(LinkRuntimeError, match="non-empty mutable query"):
        resolve_link_plan({"a": [1]}, [], {"cache_keys": ["a"]})
    with pytest.raises(LinkRuntimeError, match="one value per cache key"):
        resolve_link_plan({"a": [1]}, [2], {"cache_keys": ["a"], "recompute_tokens_per_block": [1, 2]})
    with pytest.raises(LinkRuntimeError, match="require the normalized physical token layout"):
        resolve_link_plan({"a": [1], "b": [2]}, [3], {"cache_keys": ["a", "b"],
                                                     "physical_interblock_fresh_token_counts": [1]})


def test_interblock_gaps_are_recomputed_and_shift_later_blocks():
    blocks = {"a": [10, 11], "b": [20, 21]}
    plan = {"cache_keys": ["a", "b"], "recompute_initial_tokens": 1, "physical_prefix_token_count": 1,
            "physical_interblock_fresh_token_counts": [2]}
    linked = resolve_link_plan(blocks, [100, 50, 51, 30], plan)
    assert linked == [100, 10, 11, 50, 51, 20, 21, 30]
    assert [r["start_token"] for r in plan["block_ranges"]] == [1, 5]
    assert plan["imp_indices"] == [0, 3, 4, 5, 7]


def test_registry_lookup_pin_and_evict():
    registry = LegoLinkBlockRegistry()
    handle = registry.register_legolink_block("a", [1, 2, 3], torch.tensor([7, 8, 9]))
    assert handle.compile_local_positions == (0, 1, 2)
    with pytest.raises(ValueError, match="exact logical token length"):
        registry.register_legolink_block("b", [1, 2], torch.tensor([1]))
    with pytest.raises(ValueError, match="already registered"):
        registry.register_legolink_block("a", [1], torch.tensor([1]))
    result = registry.lookup_legolink_blocks(["a", "zz"])
    assert result.missing_blocks == ["zz"] and list(result.matched_blocks) == ["a"]
    registry.acquire_legolink_blocks(result.matched_handles)
    assert registry.evict_legolink_block("a") is None  # pinned
    registry.release_legolink_blocks(result.matched_handles)
    assert registry.evict_legolink_block("a") is not None
    assert registry.lookup_legolink_blocks(["a"]).stale_blocks == ["a"]
    assert registry.get_legolink_block_tokens("a") is None
    with pytest.raises(ValueError, match="not pinned"):
        registry.release_legolink_blocks(result.matched_handles)


def _executor(blocks, *, layers=1, compile_positions=None):
    registry = LegoLinkBlockRegistry()
    slot = 100
    for key, count in blocks.items():
        positions = None if compile_positions is None else compile_positions.get(key)
        registry.register_legolink_block(key, list(range(count)), torch.arange(slot, slot + count),
                                         compile_local_positions=positions)
        slot += count
    rotary = RotarySpec.for_theta(64, 8, theta=1e4)
    return KVLinkExecutor(registry, rotary, start_layer=0, end_layer=layers)


@pytest.mark.parametrize("case", GOLDEN["first_block_remap"]["cases"], ids=lambda c: str(c["blocks"]))
def test_remap_decision_follows_the_offset(case):
    """tests/pic/test_first_block_rope_remap.py: a block is remapped iff its
    request offset differs from its compile positions, never by its ordinal."""

    blocks = {f"block-{i}": count for i, (_, count) in enumerate(case["blocks"])}
    executor = _executor(blocks)
    total = max(start + count for start, count in case["blocks"])
    plan = {"cache_keys": list(blocks),
            "block_ranges": [{"start_token": s, "end_token": s + c} for s, c in case["blocks"]]}
    maps = executor.build_link_maps(torch.arange(total), plan)
    assert [spec["needs_rope_remap"] for spec in maps.block_specs] == case["expected_remapped"]
    first_count = case["blocks"][0][1]
    assert maps.prefix_token_count == (0 if case["expected_remapped"][0] else first_count)


def test_link_maps_follow_plan_order():
    executor = _executor({"a": 3, "b": 2}, compile_positions={"b": [40, 41]})
    destination = torch.arange(500, 510)
    plan = {"cache_keys": ["b", "a"], "block_ranges": [{"start_token": 1, "end_token": 3},
                                                       {"start_token": 3, "end_token": 6}],
            "imp_indices": [0, 3, 4, 9]}
    maps = executor.build_link_maps(destination, plan)
    assert maps.source_slots.tolist() == [103, 104, 100, 101, 102]
    assert maps.destination_slots.tolist() == [501, 502, 503, 504, 505]
    assert maps.local_positions.tolist() == [40, 41, 0, 1, 2]
    assert maps.global_positions.tolist() == [1, 2, 3, 4, 5]
    assert maps.repair_offsets.tolist() == [2, 3]  # positions 3 and 4 fall inside block "a"
    assert maps.prefix_token_count == 0


def test_executor_errors():
    executor = _executor({"a": 3})
    plan = {"cache_keys": ["a", "missing"],
            "block_ranges": [{"start_token": 0, "end_token": 3}, {"start_token": 3, "end_token": 4}]}
    with pytest.raises(LinkRuntimeError, match="cannot safely link block\\(s\\): missing"):
        executor.build_link_maps(torch.arange(8), plan)
    with pytest.raises(LinkRuntimeError, match="token count mismatch for block a: plan=2, snapshot=3"):
        executor.build_link_maps(torch.arange(8), {"cache_keys": ["a"],
                                                   "block_ranges": [{"start_token": 0, "end_token": 2}]})
    with pytest.raises(LinkRuntimeError, match="counts differ"):
        executor.build_link_maps(torch.arange(8), {"cache_keys": ["a"], "block_ranges": [
            {"start_token": 0, "end_token": 3}, {"start_token": 3, "end_token": 4}]})
    with pytest.raises(LinkRuntimeError, match="missing block ranges"):
        executor.build_link_maps(torch.arange(8), {"cache_keys": ["a"], "block_ranges": []})

    class QuantizedPool:
        dtype = torch.bfloat16
        store_dtype = torch.uint8
        def get_key_buffer(self, layer): ...
        def get_value_buffer(self, layer): ...

    with pytest.raises(LinkRuntimeError, match="quantized KV cache"):
        executor.prepare_link(QuantizedPool(), torch.arange(8), {"cache_keys": ["a"]})
    with pytest.raises(LinkRuntimeError, match="MHA-style KV pool"):
        executor.prepare_link(object(), torch.arange(8), {"cache_keys": ["a"]})


def test_cpu_pool_is_rejected_loudly():
    executor = _executor({"a": 3})
    pool = KVPool.allocate(num_slots=200, num_layers=1, num_heads=2, head_dim=8, device="cpu")
    plan = {"cache_keys": ["a"], "block_ranges": [{"start_token": 2, "end_token": 5}]}
    with pytest.raises(RuntimeError, match="cuda_tensors_required"):
        executor.copy_linked_kv(pool, torch.arange(10), plan)
    # the pin taken for the link is released on failure
    assert executor.registry.lookup_legolink_blocks(["a"]).matched_handles[0].pin_count == 0


def test_snapshot_arena_allocates_and_merges_ranges():
    from legolink_amd.link_runtime import SnapshotArena

    arena = SnapshotArena([torch.zeros(10, 1, 8)], [torch.zeros(10, 1, 8)])
    a = arena.alloc(4)
    b = arena.alloc(3)
    assert a.tolist() == [0, 1, 2, 3] and b.tolist() == [4, 5, 6]
    assert arena.alloc(4) is None and arena.free_slots == 3
    arena.free(a)
    c = arena.alloc(2)
    assert c.tolist() == [0, 1]
    arena.free(b)
    arena.free(c)
    assert arena.free_slots == 10 and arena._free == [(0, 10)]
    with pytest.raises(ValueError, match="already free"):
        arena.free(torch.arange(2, 4))
    with pytest.raises(ValueError, match="range alloc returned"):
        arena.free(torch.tensor([1, 3]))


def test_storage_modes_in_registry_and_maps():
    registry = LegoLinkBlockRegistry()
    with pytest.raises(ValueError, match="Unsupported PIC storage mode"):
        registry.register_legolink_block("x", [1], torch.tensor([0]), storage_mode="paged")
    registry.register_legolink_block("r", [1, 2], torch.tensor([10, 11]))
    registry.register_legolink_block("c", [3, 4, 5], torch.tensor([0, 1, 2]), storage_mode="clone")
    executor = KVLinkExecutor(registry, RotarySpec.for_theta(16, 8, theta=1e4),
                              end_layer=1)
    plan = {"cache_keys": ["c", "r"], "block_ranges": [{"start_token": 0, "end_token": 3},
                                                       {"start_token": 3, "end_token": 5}]}
    maps = executor.build_link_maps(torch.arange(20, 25), plan)
    assert maps.clone_tokens.tolist() == [True, True, True, False, False]
    assert [spec["storage_mode"] for spec in maps.block_specs] == ["clone", "reference"]
    pool = KVPool.allocate(num_slots=32, num_layers=1, num_heads=1, head_dim=8, device="cpu")
    with pytest.raises(LinkRuntimeError, match="needs the snapshot arena"):
        executor.prepare_link(pool, torch.arange(20, 25), plan)


def test_batched_capture_rejects_before_any_registration():
    """capture_blocks checks every entry before it copies or registers one."""

    registry = LegoLinkBlockRegistry()
    executor = KVLinkExecutor(registry, RotarySpec.for_theta(16, 8, theta=1e4),
                              end_layer=1)
    pool = KVPool.allocate(num_slots=32, num_layers=1, num_heads=1, head_dim=8, device="cpu")
    reference = {"cache_key": "r", "token_ids": [1, 2], "slots": [3, 4]}
    with pytest.raises(LinkRuntimeError, match="needs a snapshot arena"):
        executor.capture_blocks(pool, [reference, {"cache_key": "c", "token_ids": [5], "slots": [6],
                                                   "storage_mode": "clone"}])
    with pytest.raises(LinkRuntimeError, match="Unsupported PIC storage mode"):
        executor.capture_blocks(pool, [reference, {"cache_key": "p", "token_ids": [5], "slots": [6],
                                                   "storage_mode": "paged"}])
    assert registry.get_legolink_block_tokens("r") is None
    # A reference-only batch needs no copy and registers every entry.
    handles = executor.capture_blocks(pool, [reference, {"cache_key": "s", "token_ids": [7], "slots": [8],
                                                         "block_id": "seg"}])
    assert [handle.cache_key for handle in handles] == ["r", "s"]
    assert handles[0].kv_slots.tolist() == [3, 4] and handles[1].block_id == "seg"
    with pytest.raises(ValueError, match="slot count"):
        executor.capture_blocks(pool, [{"cache_key": "t", "token_ids": [1, 2, 3], "slots": [0]}])
    assert registry.get_legolink_block_tokens("t") is None
    # A key registered twice in one batch: the entries before it are evicted again.
    with pytest.raises(ValueError, match="already registered"):
        executor.capture_blocks(pool, [{"cache_key": "u", "token_ids": [1], "slots": [9]},
                                       {"cache_key": "u", "token_ids": [2], "slots": [10]}])
    assert registry.get_legolink_block_tokens("u") is None
    assert registry.get_legolink_block_tokens("r") == (1, 2)  # earlier blocks untouched


def test_visit_order_defaults_and_validation():
    from legolink_amd.link_runtime import _resolve_visit_order

    assert _resolve_visit_order(None, None, 1) == "destination"
    assert _resolve_visit_order(None, None, 4) == "source"
    assert _resolve_visit_order(None, False, 4) == "plan"
    assert _resolve_visit_order(None, True, 1) == "source"
    assert _resolve_visit_order("plan", True, 4) == "plan"
    with pytest.raises(ValueError, match="visit_order"):
        _resolve_visit_order("random", None, 1)
    with pytest.raises(ValueError, match="visit_order"):
        KVLinkExecutor(LegoLinkBlockRegistry(), RotarySpec.for_theta(64, 64), end_layer=1, visit_order="sideways")


def test_registry_rows_are_reused_after_eviction():
    """Registering and evicting blocks over and over keeps the per-device record
    table as large as the most blocks live at once, and an evicted handle's
    device copies are released."""

    registry = LegoLinkBlockRegistry()
    cpu = torch.device("cpu")
    live = []
    for index in range(2000):
        handle = registry.register_legolink_block(f"k{index}", range(4), torch.arange(4 * index, 4 * index + 4))
        records = registry.link_records([handle], cpu)
        assert records[0, 0] == 4 and records[0, 4] == 0
        live.append(handle)
        if len(live) > 5:
            old = live.pop(0)
            assert registry.evict_legolink_block(old.cache_key) is old
            assert old.row == -1 and not old._device_tensors
    assert registry.record_rows <= 6
    table, _ = registry._records[(cpu.type, cpu.index)]
    assert table.shape[0] <= 64
    # A reused row holds the new handle's record, not the evicted one's.
    again = registry.register_legolink_block("again", range(9), torch.arange(9))
    assert registry.link_records([again], cpu)[0, 0] == 9
    assert registry.lookup_legolink_blocks(["k0"]).stale_blocks == ["k0"]
    with pytest.raises(ValueError, match="evicted"):
        registry.link_records([registry._blocks["k0"]], cpu)
