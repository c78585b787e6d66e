"""Token maps of a link (no GPU): the oracle pinned to the reference's cases,
the host run planner checked against the oracle through the map builder's
documented semantics, and the C entry's argument validation."""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

from legolink_amd import _native, link_maps
from oracle import link_maps_oracle as lmo

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
F = {name: index for index, name in enumerate(_native.SEGMENT_FIELDS)}

# Repair rows inside blocks (concatenation offsets) and identity prefix of the
# reference's plan-derivation cases, derived by hand from the reference's rule
# (pic_runtime.py:4981-4990: offset + position - start for start <= position < end;
# :5005-5013: block 0's count when block 0 starts at position 0).
EXPECTED = {
    "legacy_two_blocks": ([3], 3),          # imp [3, 5, 6]: 3 opens block b; 5, 6 are the suffix
    "normalized_chat_prefix": ([3], 0),     # blocks at 1 and 4; imp [0, 4, 6, 7]: only 4 is inside
    "recompute_first_block": ([0, 3], 3),   # imp [0, 3, 5, 6]
    "per_block_recompute_counts": ([0, 1, 3], 3),  # imp [0, 1, 3, 6]
    "trace_offsets": ([2], 2),              # blocks at 0 and 2; imp [2, 4]
}


def _golden_blocks(case):
    lengths = [len(case["blocks"][key]) for key in case["cache_keys"]]
    if "expected_block_ranges" in case:
        starts = [r["start_token"] for r in case["expected_block_ranges"]]
    elif "expected_block_starts" in case:
        starts = case["expected_block_starts"]
    else:
        starts = list(np.concatenate(([0], np.cumsum(lengths)[:-1])))
    return [{"start": int(s), "source_slots": np.arange(n) + 50 * i, "local_positions": np.arange(n), "set": 0}
            for i, (s, n) in enumerate(zip(starts, lengths))]


@pytest.mark.parametrize("case", GOLDEN["plan_derivation"]["cases"], ids=lambda c: c["name"])
def test_oracle_repair_rows_and_prefix_on_reference_plans(case):
    blocks = _golden_blocks(case)
    request_slots = np.arange(40) + 100
    whole = lmo.concatenated_maps(blocks, request_slots, case["expected_imp_indices"])
    offsets, prefix = EXPECTED[case["name"]]
    assert whole["repair_offsets"].tolist() == offsets
    assert whole["prefix_token_count"] == prefix


def test_oracle_on_the_reference_two_block_link():
    # test_sglang_pic_runtime.py:864-913: blocks a, b of 2 tokens at 0 and 2, destination [4, 5, 6, 7].
    blocks = [{"start": 0, "source_slots": np.array([9, 3]), "local_positions": np.array([0, 1]), "set": 0},
              {"start": 2, "source_slots": np.array([6, 1]), "local_positions": np.array([0, 1]), "set": 0}]
    whole = lmo.concatenated_maps(blocks, np.array([4, 5, 6, 7]), [])
    assert whole["destination_slots"].tolist() == [4, 5, 6, 7]
    assert whole["global_positions"].tolist() == [0, 1, 2, 3]
    assert whole["local_positions"].tolist() == [0, 1, 0, 1]
    assert whole["source_slots"].tolist() == [9, 3, 6, 1]
    assert whole["prefix_token_count"] == 2


@pytest.mark.parametrize("case", GOLDEN["first_block_remap"]["cases"], ids=str)
def test_oracle_prefix_follows_the_first_block_rule(case):
    # tests/pic/test_first_block_rope_remap.py:126-249: blocks [start, count], compiled at 0..n-1.
    blocks = [{"start": s, "source_slots": np.arange(n), "local_positions": np.arange(n), "set": 0}
              for s, n in case["blocks"]]
    whole = lmo.concatenated_maps(blocks, np.arange(64), [])
    first_count = case["blocks"][0][1]
    assert whole["prefix_token_count"] == (0 if case["expected_remapped"][0] else first_count)


def _random_plan(rng, *, blocks=None, max_len=40, clone_fraction=0.3, non_affine_fraction=0.2):
    count = int(rng.integers(1, 12)) if blocks is None else blocks
    lengths = rng.integers(1, max_len, size=count)
    gaps = rng.integers(0, 4, size=count)
    order = rng.permutation(count)  # plan order differs from position order
    starts = np.empty(count, dtype=np.int64)
    cursor = int(rng.integers(0, 3))
    for b in range(count):
        starts[b] = cursor
        cursor += int(lengths[b] + gaps[b])
    total = cursor + 5
    plan_blocks = []
    for b in order:
        n = int(lengths[b])
        if rng.random() < non_affine_fraction:
            local = rng.integers(0, 5000, size=n)
        else:
            local = int(rng.integers(0, 3000)) + np.arange(n)
        if b == order[0] and rng.random() < 0.4:
            local = int(starts[b]) + np.arange(n)  # an identity first block
        plan_blocks.append({"start": int(starts[b]), "source_slots": rng.integers(0, 10**6, size=n),
                            "local_positions": np.asarray(local, dtype=np.int64),
                            "set": int(rng.random() < clone_fraction)})
    imp = rng.integers(0, total, size=int(rng.integers(0, total // 2 + 1))).tolist()
    # Runs that span block seams and repeated positions.
    for b in range(count):
        if rng.random() < 0.5:
            seam = int(starts[b])
            imp.extend(range(max(0, seam - 2), seam + int(rng.integers(1, 6))))
    return plan_blocks, np.arange(total, dtype=np.int64) * 7 + 3, imp


def _characterize(blocks, request_slots, imp, out):
    """What the maps must satisfy, independent of how they are built."""

    imp_set = set(int(p) for p in imp)
    token_global = np.concatenate([b["start"] + np.arange(len(b["source_slots"])) for b in blocks])
    repair_tokens = {t for t, g in enumerate(token_global) if int(g) in imp_set}
    assert set(out["repair_offsets"].tolist()) == repair_tokens
    assert list(out["repair_offsets"]) == sorted(out["repair_offsets"])
    assert np.array_equal(out["destination_slots"], request_slots[out["global_positions"]])
    assert np.array_equal(out["global_positions"], token_global)


def test_oracle_maps_satisfy_the_characterization_and_a_planted_mistake_fails():
    rng = np.random.default_rng(7)
    for _ in range(50):
        blocks, request_slots, imp = _random_plan(rng)
        _characterize(blocks, request_slots, imp, lmo.concatenated_maps(blocks, request_slots, imp))
    # A plausible slip: repair offsets taken relative to the request, not the concatenation.
    blocks, request_slots, imp = _random_plan(np.random.default_rng(3), blocks=6)
    out = lmo.concatenated_maps(blocks, request_slots, imp)
    wrong = dict(out)
    wrong["repair_offsets"] = np.asarray(sorted(p for p in set(imp) if p < out["global_positions"].size))
    with pytest.raises(AssertionError):
        _characterize(blocks, request_slots, imp, wrong)


def _fake_table(blocks):
    """Block table whose 'device addresses' name host arrays: block i's slots at
    (i + 1) << 32, its explicit local positions at (i + 1001) << 32."""

    arrays = {}
    starts, counts, sources, locals_, local_starts, sets = [], [], [], [], [], []
    for i, block in enumerate(blocks):
        n = len(block["source_slots"])
        arrays[i + 1] = np.asarray(block["source_slots"], dtype=np.int64)
        local = np.asarray(block["local_positions"], dtype=np.int64)
        affine = n == 0 or np.array_equal(local, local[0] + np.arange(n))
        starts.append(block["start"])
        counts.append(n)
        sources.append((i + 1) << 32)
        if affine:
            locals_.append(0)
            local_starts.append(int(local[0]) if n else 0)
        else:
            arrays[i + 1001] = local
            locals_.append((i + 1001) << 32)
            local_starts.append(0)
        sets.append(block["set"])
    return link_maps.block_table(starts, counts, sources, locals_, local_starts, sets), arrays


def _apply_segments(table, arrays, request_slots, map_counts, repair_count, compact):
    """The builder's semantics as the C header states them, on host arrays."""

    maps = [np.full((4, n), -1, dtype=np.int64) for n in map_counts]
    masks = [None if compact else np.full(n, 255, dtype=np.uint8) for n in map_counts]
    repair = np.full(repair_count, -1, dtype=np.int64)
    deref = lambda address, i: arrays[address >> 32][((address & 0xFFFFFFFF) >> 3) + i]
    for row in table:
        for i in range(int(row[F["token_count"]])):
            p = int(row[F["start_token"]]) + i
            d = int(request_slots[int(row[F["destination_start"]]) + i])
            is_repair = row[F["repair_begin"]] <= i < row[F["repair_end"]]
            if is_repair and row[F["repair_offset"]] >= 0:
                repair[row[F["repair_offset"]] + i - row[F["repair_begin"]]] = d
            s = int(row[F["map_set"]])
            if is_repair and masks[s] is None:
                continue
            o = int(row[F["map_offset"]]) + i
            if masks[s] is None and i >= row[F["repair_end"]]:
                o -= int(row[F["repair_end"]] - row[F["repair_begin"]])
            local = (deref(int(row[F["local_positions"]]), i) if row[F["local_positions"]]
                     else int(row[F["local_start"]]) + i)
            maps[s][:, o] = (deref(int(row[F["source_slots"]]), i), d, local, p)
            if masks[s] is not None:
                masks[s][o] = 1 if is_repair else 0
    return maps, masks, repair


@pytest.mark.parametrize("compact", [True, False])
def test_planner_runs_reproduce_the_oracle_maps(compact):
    rng = np.random.default_rng(11 if compact else 12)
    for trial in range(60):
        blocks, request_slots, imp = _random_plan(rng, max_len=70 if trial % 3 == 0 else 20)
        table, arrays = _fake_table(blocks)
        plan = link_maps.plan_segments(table, np.asarray(imp, dtype=np.int64), compact=compact)
        assert (plan.table[:, F["repair_end"]] - plan.table[:, F["repair_begin"]] >= 0).all()
        maps, masks, repair = _apply_segments(plan.table, arrays, request_slots, plan.map_counts,
                                              plan.repair_count, compact)
        expected = lmo.device_maps(blocks, request_slots, imp, compact=compact)
        assert np.array_equal(plan.repair_offsets, expected["repair_offsets"])
        assert np.array_equal(repair, expected["repair_destination_slots"])
        for s in (0, 1):
            if expected[f"maps{s}"] is None:
                assert plan.map_counts[s] == 0
                continue
            assert np.array_equal(maps[s], expected[f"maps{s}"]), (trial, s)
            if not compact:
                assert np.array_equal(masks[s], expected[f"mask{s}"])
        first_set = blocks[0]["set"]
        assert expected[f"prefix{first_set}"] == (int(plan.block_entries[0])
                                                  if expected["prefix_token_count"] else 0)


def test_planner_batches_requests_like_the_oracle():
    rng = np.random.default_rng(21)
    for trial in range(30):
        compact = bool(trial % 2)
        requests = []
        for _ in range(int(rng.integers(2, 6))):
            blocks, slots, imp = _random_plan(rng, max_len=25)
            requests.append((blocks, slots, imp))
        tables, bases, leading, repairs, arrays = [], [], [], [], {}
        base = 0
        for r, (blocks, slots, imp) in enumerate(requests):
            # Distinct fake addresses per request: shift the block ids.
            shifted = [dict(b) for b in blocks]
            table, block_arrays = _fake_table(shifted)
            table.source_ptrs = table.source_ptrs + ((r * 50) << 32)
            table.local_ptrs = np.where(table.local_ptrs != 0, table.local_ptrs + ((r * 50) << 32), 0)
            arrays.update({key + r * 50: value for key, value in block_arrays.items()})
            tables.append(table)
            bases.append(base)
            whole = lmo.concatenated_maps(blocks, slots, imp)
            lead = np.zeros(len(blocks), dtype=bool)
            lead[0] = whole["prefix_token_count"] > 0
            leading.append(lead)
            repairs.append(np.asarray(imp, dtype=np.int64) + base)
            base += slots.size
        batched = link_maps.concatenate_tables(tables, bases)
        plan = link_maps.plan_segments(batched, np.concatenate(repairs), compact=compact,
                                       leading_blocks=np.concatenate(leading))
        all_slots = np.concatenate([slots for _, slots, _ in requests])
        maps, masks, repair = _apply_segments(plan.table, arrays, all_slots, plan.map_counts,
                                              plan.repair_count, compact)
        expected = lmo.batched_device_maps(requests, compact=compact)
        assert np.array_equal(repair, expected["repair_destination_slots"]), trial
        for s in (0, 1):
            assert plan.set_prefix[s] == expected[f"prefix{s}"]
            if expected[f"maps{s}"] is None:
                assert plan.map_counts[s] == 0
                continue
            assert np.array_equal(maps[s], expected[f"maps{s}"]), (trial, s)
            if not compact:
                assert np.array_equal(masks[s], expected[f"mask{s}"])


def test_planner_cuts_a_block_per_repair_run():
    table = link_maps.block_table([0, 10], [10, 6], [1 << 32, 2 << 32], [0, 0], [0, 0], [0, 0])
    plan = link_maps.plan_segments(table, np.array([10, 11, 3, 4, 7]), compact=True)
    rows = [(r[F["start_token"]], r[F["token_count"]], r[F["repair_begin"]], r[F["repair_end"]],
             r[F["map_offset"]]) for r in plan.table]
    # Block 0: runs [3, 5) and [7, 8) -> runs [0, 7) and [7, 10); block 1: run [10, 12) -> one run.
    assert rows == [(0, 7, 3, 5, 0), (7, 3, 0, 1, 5), (10, 6, 0, 2, 7)]
    assert plan.map_counts == (11, 0) and plan.repair_count == 5
    assert plan.repair_offsets.tolist() == [3, 4, 7, 10, 11]


def _maps_args(table, *, dest=16, capacity=(64, 0), repair_capacity=8, dtype=_native.DTYPE_INT64):
    args = _native.LinkMapsArgs()
    args.num_segments = table.shape[0]
    args.segments = table.ctypes.data
    args.destination_slots = 0x1000
    args.destination_slots_dtype = dtype
    args.num_destination_slots = dest
    args.maps[0] = 0x2000
    args.map_capacity[0], args.map_capacity[1] = capacity
    args.repair_destination_slots = 0x3000
    args.repair_capacity = repair_capacity
    return args


def _segment(**fields):
    row = np.zeros((1, len(F)), dtype=np.int64)
    row[0, F["source_slots"]] = 0x4000
    row[0, F["token_count"]] = 4
    for name, value in fields.items():
        row[0, F[name]] = value
    return row


@pytest.mark.parametrize("fields,kwargs,message", [
    (dict(destination_start=14), {}, "outside the 16 destination slots"),
    (dict(start_token=-1), {}, "start_token out of range"),
    (dict(map_set=2), {}, "map_set must be 0 or 1"),
    (dict(map_set=1), {}, "maps[1] is NULL"),
    (dict(map_offset=62), {}, "outside capacity 64"),
    (dict(repair_begin=1, repair_end=3, repair_offset=7), {}, "outside capacity 8"),
    (dict(repair_begin=3, repair_end=2), {}, "repair rows outside the run"),
    (dict(token_count=-1), {}, "token_count out of range"),
    (dict(source_slots=0), {}, "source_slots is NULL"),
    (dict(repair_offset=-2), {}, "repair_offset must be >= -1"),
    ({}, dict(dtype=_native.DTYPE_FLOAT32), "int32 or int64"),
])
def test_map_builder_rejects_bad_runs_before_any_launch(fields, kwargs, message):
    table = _segment(**fields)
    args = _maps_args(table, **kwargs)
    with pytest.raises(_native.NativeCallError) as error:
        _native.kv_build_link_maps(args, 0)
    assert message in str(error.value)


def test_map_builder_struct_checks():
    lib = _native.load_library()
    assert lib.ll_link_maps_args_size() == ctypes.sizeof(_native.LinkMapsArgs)
    assert ctypes.sizeof(_native.LinkSegment) == 8 * len(F)
    assert lib.ll_kv_build_link_maps(None, None) == _native.LL_ERR_INVALID_ARGUMENT
    args = _maps_args(_segment())
    args.struct_size = 8
    assert lib.ll_kv_build_link_maps(ctypes.byref(args), None) == _native.LL_ERR_INVALID_ARGUMENT
    empty = _native.LinkMapsArgs()
    _native.kv_build_link_maps(empty, 0)  # no runs: nothing to do, no GPU touched


def test_order_entry_rejects_bad_arguments_before_any_launch():
    """ll_order_link_maps checks its arguments on the host (no GPU here: every
    case returns before a launch)."""

    lib = _native.load_library()
    assert lib.ll_order_link_maps(None, None) == _native.LL_ERR_INVALID_ARGUMENT

    def args(**fields):
        a = _native.OrderMapsArgs()
        a.struct_size = ctypes.sizeof(a)
        a.maps, a.out_maps, a.workspace = 0x100000, 0x200000, 0x300000
        a.capacity = a.count = 100
        a.prefix, a.num_slots = 10, 1000
        a.workspace_bytes = _native.ORDER_WORKSPACE_BYTES
        a.key_row = 1
        for key, value in fields.items():
            setattr(a, key, value)
        return a

    for fields, message in [
        (dict(struct_size=8), "struct_size"),
        (dict(count=101), "prefix <= count <= capacity"),
        (dict(prefix=101), "prefix <= count"),
        (dict(capacity=1 << 31, count=1 << 31), "2^31"),
        (dict(num_slots=0), "num_slots"),
        (dict(maps=None), "device arrays"),
        (dict(mask=0x400000), "both"),
        (dict(out_maps=0x100000 + 8 * 399), "overlaps"),
        (dict(maps=0x100004), "aligned"),
        (dict(mask=0x400000, out_mask=0x400000 + 50), "out_mask overlaps"),
        (dict(workspace_bytes=_native.ORDER_WORKSPACE_BYTES - 1), "workspace"),
        (dict(workspace=None), "workspace"),
        (dict(workspace=0x300008), "16-byte aligned"),
        (dict(key_row=2), "key_row"),
        (dict(key_row=-1), "key_row"),
    ]:
        status = lib.ll_order_link_maps(ctypes.byref(args(**fields)), None)
        assert status == _native.LL_ERR_INVALID_ARGUMENT, fields
        assert message in lib.ll_last_error().decode(), (fields, lib.ll_last_error())
    assert lib.ll_order_link_maps(ctypes.byref(args(count=0, prefix=0)), None) == _native.LL_OK  # nothing to do
