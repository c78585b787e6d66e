"""Hostile and undersized inputs to the library's host entries (CPU, no GPU).

Every case here returns before any HIP call: the run planner and the repair
attention planner are host-only, and the link, map-builder and attention
entries reject these arguments before they launch.  The same tests run
against the host-sanitized build (test_host_sanitizer.py), where an
out-of-bounds access or undefined behaviour fails them.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from legolink_amd import _native

FIELDS = {name: index for index, name in enumerate(_native.SEGMENT_FIELDS)}
BLOCK = {name: index for index, name in enumerate(_native.BLOCK_FIELDS)}


def _blocks(rows):
    """int64 [B, 8] block records from (start, count, base, set, leading) tuples."""

    table = np.zeros((len(rows), len(BLOCK)), dtype=np.int64)
    for index, (start, count, base, map_set, leading) in enumerate(rows):
        table[index, BLOCK["source_slots"]] = 0x10000 + 0x1000 * index
        table[index, BLOCK["token_count"]] = count
        table[index, BLOCK["start_token"]] = start
        table[index, BLOCK["destination_base"]] = base
        table[index, BLOCK["local_start"]] = 3 * index
        table[index, BLOCK["map_set"]] = map_set
        table[index, BLOCK["leading"]] = leading
    return table


def _brute_force(blocks, positions, compact):
    """Per token, in plan order: (block, offset, is repair row); then the map
    entries of each set (leading blocks first) and the repair offsets."""

    wanted = set(int(p) for p in positions)
    tokens, concat = [], 0
    for b, row in enumerate(blocks):
        dstart = row[BLOCK["start_token"]] + row[BLOCK["destination_base"]]
        for i in range(row[BLOCK["token_count"]]):
            tokens.append((b, i, (dstart + i) in wanted, concat + i))
        concat += row[BLOCK["token_count"]]
    repair_offsets = [c for _, _, repair, c in tokens if repair]
    entries = {0: [], 1: []}
    for lead in (1, 0):
        for b, i, repair, _ in tokens:
            row = blocks[b]
            if row[BLOCK["leading"]] == lead and not (compact and repair):
                entries[int(row[BLOCK["map_set"]])].append((b, i))
    return entries, repair_offsets


def _planned_entries(blocks, table, compact):
    """The map entries the planned runs produce, per set, in map order."""

    entries = {0: {}, 1: {}}
    by_source = {int(row[BLOCK["source_slots"]]): b for b, row in enumerate(blocks)}
    for run in table:
        b = max(k for k in by_source if k <= run[FIELDS["source_slots"]])
        block = by_source[b]
        first = (run[FIELDS["source_slots"]] - b) // 8
        rb, re = run[FIELDS["repair_begin"]], run[FIELDS["repair_end"]]
        cursor = run[FIELDS["map_offset"]]
        for i in range(run[FIELDS["token_count"]]):
            if compact and rb <= i < re:
                continue
            entries[int(run[FIELDS["map_set"]])][cursor] = (block, first + i)
            cursor += 1
    return {s: [entries[s][k] for k in sorted(entries[s])] for s in (0, 1)}


@pytest.mark.parametrize("seed", range(12))
def test_run_planner_fuzz_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    rows, start = [], 0
    for _ in range(int(rng.integers(1, 12))):
        count = int(rng.integers(0, 40))
        rows.append((start, count, int(rng.integers(0, 3)) * 1000, int(rng.integers(0, 2)), int(rng.random() < 0.2)))
        start += count + int(rng.integers(0, 5))
    if seed % 3 == 0:  # blocks out of position order (several requests' bases)
        rows = rows[::-1]
    blocks = _blocks(rows)
    top = max(r[0] + r[1] + r[2] for r in rows) + 10
    positions = rng.integers(-5, top + 50, size=int(rng.integers(0, 120)))  # unsorted, duplicates, outside
    compact = bool(seed % 2)
    table, segment_blocks, repair_offsets, info = _native.plan_link_runs(blocks, positions, compact)
    entries, expected_repairs = _brute_force(blocks, positions, compact)
    assert repair_offsets.tolist() == expected_repairs
    assert info.repair_count == len(expected_repairs)
    assert _planned_entries(blocks, table, compact) == entries
    assert [int(info.map_count[s]) for s in (0, 1)] == [len(entries[s]) for s in (0, 1)]
    # Runs cover every token of every block once, in plan order.
    covered = {}
    for run, b in zip(table, segment_blocks):
        first = (run[FIELDS["source_slots"]] - blocks[b, BLOCK["source_slots"]]) // 8
        for i in range(run[FIELDS["token_count"]]):
            key = (int(b), int(first + i))
            assert key not in covered
            covered[key] = True
    assert len(covered) == sum(r[1] for r in rows)


@pytest.mark.parametrize("seed", range(16))
def test_run_planner_matches_brute_force_on_position_runs(seed):
    """Repair positions in runs (a seam's imp_indices) that start before,
    cross and end after block boundaries, increasing or shuffled with
    repeats, and the largest and smallest int64 positions."""

    rng = np.random.default_rng([7, seed])
    rows, start = [], 0
    for _ in range(int(rng.integers(1, 14))):
        count = int(rng.integers(0, 48))
        rows.append((start, count, 0, int(rng.integers(0, 2)), int(rng.random() < 0.2)))
        start += count + int(rng.integers(0, 4))
    if seed % 4 == 3:
        rows = rows[::-1]
    blocks = _blocks(rows)
    runs, cursor = [], int(rng.integers(-6, 6))
    while cursor < start + 8:
        length = int(rng.integers(1, 40))
        runs.extend(range(cursor, cursor + length))
        cursor += length + int(rng.integers(1, 20))
    positions = np.array(runs + [(1 << 63) - 1, -(1 << 63)] if seed % 2 else runs, dtype=np.int64)
    if seed % 3 == 0:
        positions = np.concatenate([positions, positions[: positions.size // 4]])
        rng.shuffle(positions)
    elif seed % 2:
        positions = np.sort(positions)
    compact = bool(seed % 5 != 0)
    table, segment_blocks, repair_offsets, info = _native.plan_link_runs(blocks, positions, compact)
    entries, expected_repairs = _brute_force(blocks, positions, compact)
    assert repair_offsets.tolist() == expected_repairs
    assert _planned_entries(blocks, table, compact) == entries


def _raw_plan(blocks, positions, *, segment_capacity, repair_capacity, count=None, positions_count=None):
    lib = _native.load_library()
    blocks = np.ascontiguousarray(blocks, dtype=np.int64)
    positions = np.ascontiguousarray(positions, dtype=np.int64)
    segments = np.zeros((max(segment_capacity, 1), len(FIELDS)), dtype=np.int64)
    segment_blocks = np.zeros(max(segment_capacity, 1), dtype=np.int64)
    repairs = np.zeros(max(repair_capacity, 1), dtype=np.int64)
    info = _native.LinkRunPlanInfo()
    status = lib.ll_plan_link_runs(
        blocks.ctypes.data if blocks.size else None, blocks.shape[0] if count is None else count,
        positions.ctypes.data if positions.size else None,
        positions.size if positions_count is None else positions_count, 1,
        segments.ctypes.data, segment_capacity, segment_blocks.ctypes.data, repairs.ctypes.data,
        repair_capacity, ctypes.byref(info))
    return status, lib.ll_last_error().decode(), info


def test_run_planner_rejects_hostile_blocks_and_small_outputs():
    good = _blocks([(0, 10, 0, 0, 0), (10, 5, 0, 1, 0)])
    status, message, info = _raw_plan(good, [3, 4, 11], segment_capacity=16, repair_capacity=16)
    assert status == _native.LL_OK and info.num_segments == 2  # one repair range per block
    # Undersized outputs are reported, nothing is written past them.
    status, message, _ = _raw_plan(good, [3, 4, 11], segment_capacity=1, repair_capacity=16)
    assert status == _native.LL_ERR_INVALID_ARGUMENT and "segment_capacity" in message
    status, message, _ = _raw_plan(good, [3, 4, 11], segment_capacity=16, repair_capacity=2)
    assert status == _native.LL_ERR_INVALID_ARGUMENT and "repair_offsets_capacity" in message
    for rows in ([(0, -1, 0, 0, 0)], [(0, 4, 0, 2, 0)], [(-3, 4, 0, 0, 0)], [(0, 4, -1, 0, 0)],
                 [(0, 1 << 31, 0, 0, 0)], [(1 << 62, 4, 1 << 62, 0, 0)]):
        status, message, _ = _raw_plan(_blocks(rows), [1], segment_capacity=8, repair_capacity=8)
        assert status == _native.LL_ERR_INVALID_ARGUMENT and "block 0" in message, rows
    # Counts without arrays.
    status, _, _ = _raw_plan(np.zeros((0, 8)), [1], segment_capacity=8, repair_capacity=8, count=3)
    assert status == _native.LL_ERR_INVALID_ARGUMENT
    status, _, _ = _raw_plan(good, [], segment_capacity=8, repair_capacity=8, positions_count=5)
    assert status == _native.LL_ERR_INVALID_ARGUMENT
    # Extreme positions are simply outside every block.
    status, _, info = _raw_plan(good, [-(1 << 62), 1 << 62, -1], segment_capacity=8, repair_capacity=8)
    assert status == _native.LL_OK and info.repair_count == 0


def _repair_plan_raw(rows, *, items_capacity, combine_capacity, positions_capacity, split=64):
    lib = _native.load_library()
    rows = np.ascontiguousarray(rows, dtype=np.int64).reshape(-1, 4)
    items = np.zeros((max(items_capacity, 1), _native.REPAIR_ITEM_INTS), dtype=np.int32)
    combine = np.zeros((max(combine_capacity, 1), 4), dtype=np.int32)
    positions = np.zeros(max(positions_capacity, 1), dtype=np.int32)
    info = _native.RepairPlanInfo()
    status = lib.ll_repair_attention_plan(rows.ctypes.data, rows.shape[0], 28, 4, split, items.ctypes.data,
                                          items_capacity, combine.ctypes.data, combine_capacity,
                                          positions.ctypes.data, positions_capacity, ctypes.byref(info))
    return status, lib.ll_last_error().decode(), info


def test_repair_plan_reports_undersized_tables():
    rows = [(0, 700, 16, 0), (16, 1400, 16, 0), (32, 90, 5, 3000)]
    status, _, info = _repair_plan_raw(rows, items_capacity=64, combine_capacity=64, positions_capacity=64)
    assert status == _native.LL_OK and info.num_combine > 0
    status, message, _ = _repair_plan_raw(rows, items_capacity=info.num_items - 1, combine_capacity=64,
                                          positions_capacity=64)
    assert status == _native.LL_ERR_INVALID_ARGUMENT and "items_capacity" in message
    status, message, _ = _repair_plan_raw(rows, items_capacity=64, combine_capacity=info.num_combine - 1,
                                          positions_capacity=64)
    assert status == _native.LL_ERR_INVALID_ARGUMENT and "combine_capacity" in message
    status, message, _ = _repair_plan_raw(rows, items_capacity=64, combine_capacity=64, positions_capacity=36)
    assert status == _native.LL_ERR_INVALID_ARGUMENT and "positions_capacity" in message


@pytest.mark.parametrize("row", [(0, 2**31 - 2, 5, 0), (2**31 - 3, 0, 5, 0), (0, 5, 3, 2**31 - 4),
                                 (-1, 0, 3, 0), (0, 0, -3, 0), (0, 0, 3, -1)])
def test_repair_plan_rejects_rows_that_overflow_int32(row):
    status, message, _ = _repair_plan_raw([row], items_capacity=8, combine_capacity=8, positions_capacity=64)
    assert status == _native.LL_ERR_INVALID_ARGUMENT and "row 0" in message


def test_link_describe_rejects_hostile_shapes():
    from tests.test_native_abi import _cpu_args

    for field, value in (("num_tokens", 1 << 40), ("prefix_token_count", 9), ("delta_staging", 4),
                         ("waves_per_block", 16), ("rounding", 2), ("layers_per_wave", -1),
                         ("num_layers", 0), ("key_head_dim", 300), ("cos_sin_cols", 4)):
        args, keepalive = _cpu_args()
        setattr(args, field, value)
        with pytest.raises(_native.NativeCallError):
            _native.kv_link_describe(args)
        del keepalive


def test_allocation_free_attention_rejects_before_any_launch():
    lib = _native.load_library()
    args = _native.RepairAttentionArgs()
    args.struct_size = ctypes.sizeof(args)
    args.query, args.output, args.key_buffer, args.value_buffer = 0x1000, 0x2000, 0x3000, 0x4000
    args.num_queries, args.num_slots, args.num_q_heads, args.num_kv_heads, args.head_dim = 16, 64, 28, 4, 128
    args.kv_dtype, args.softmax_scale = _native.DTYPE_BFLOAT16, 0.088
    args.kv_slots, args.kv_slots_dtype, args.kv_slots_len = 0x5000, _native.DTYPE_INT64, 64
    args.items, args.num_items, args.query_positions = 0x6000, 1, 0x7000
    args.combine, args.num_combine = 0x8000, 1
    args.workspace, args.workspace_items = 0x9000, 1  # a workspace is not taken
    assert lib.ll_repair_attention_noalloc(ctypes.byref(args), None) == _native.LL_ERR_INVALID_ARGUMENT
    args.workspace = None
    args.workspace_items = 1 << 40  # beyond the scratch array
    assert lib.ll_repair_attention_noalloc(ctypes.byref(args), None) == _native.LL_ERR_INVALID_ARGUMENT
    assert "scratch" in lib.ll_last_error().decode()
    args.num_items = 0
    args.workspace_items = 0
    assert lib.ll_repair_attention_noalloc(ctypes.byref(args), None) == _native.LL_OK  # nothing to do


def test_link_rejects_a_misaligned_counter_and_a_counter_on_an_empty_pool():
    from tests.test_native_abi import _cpu_args

    args, keepalive = _cpu_args()
    args.skipped_rows = 0x1004  # not 8-byte aligned
    with pytest.raises(_native.NativeCallError, match="aligned"):
        _native.kv_link_describe(args)
    lib = _native.load_library()
    args.skipped_rows = 0x1008
    args.num_slots = 0  # nothing would run to count the skipped tokens
    args.source_num_slots = 0
    assert lib.ll_kv_link(ctypes.byref(args), None) == _native.LL_ERR_INVALID_ARGUMENT
    assert "no rows" in lib.ll_last_error().decode()
    del keepalive
