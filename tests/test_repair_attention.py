"""Sparse repair attention without a GPU: the oracle pinned to the reference's
cases and closed forms, the host planner's coverage, and the C entry's
argument validation."""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from legolink_amd import _native
from oracle import attention_oracle as ao


def _visible_slots(slots, start, end):
    mask = ao.logical_causal_mask(np.arange(start, end), np.arange(end))
    slots = np.asarray(slots)[:end]
    return [slots[row].tolist() for row in mask]


def test_gqa_head_mapping_is_query_head_divided_by_group_size():
    # tests/pic/test_sparse_attention_reference.py:46-52
    query = np.zeros((1, 4, 2))
    key = np.zeros((1, 2, 2))
    value = np.array([[[10.0, 11.0], [20.0, 21.0]]])
    out = ao.gqa_attention(query, key, value, np.ones((1, 1), dtype=bool))
    assert out[0, :, 0].tolist() == [10.0, 10.0, 20.0, 20.0]


def test_physical_slots_never_define_logical_causal_order():
    # tests/pic/test_sparse_attention_mask.py:21-33 with the scrambled-slot fixture
    # (tests/pic/reference/fixtures.py:6-9).
    assert _visible_slots([100, 5, 80, 12], 2, 4) == [[100, 5, 80], [100, 5, 80, 12]]


def test_visibility_keeps_order_and_multiplicity():
    # tests/pic/test_sparse_attention_mask.py:36-43
    assert _visible_slots([9, 3, 9, 17, 2], 3, 5) == [[9, 3, 9, 17], [9, 3, 9, 17, 2]]


def test_physical_slot_gather_reconstructs_logical_attention():
    # tests/pic/test_sparse_attention_reference.py:12-43
    rng = np.random.default_rng(20260824)
    query = rng.standard_normal((2, 4, 8))
    logical_key = rng.standard_normal((4, 2, 8))
    logical_value = rng.standard_normal((4, 2, 8))
    slots = np.array([11, 2, 19, 7])
    key_pool = np.zeros((24, 2, 8))
    value_pool = np.zeros((24, 2, 8))
    key_pool[slots] = logical_key
    value_pool[slots] = logical_value
    expected = ao.gqa_attention(query, logical_key, logical_value,
                                ao.logical_causal_mask(np.array([2, 3]), np.arange(4)))
    actual = ao.repair_attention(query, key_pool, value_pool, slots, 2, 4)
    assert np.allclose(actual, expected, rtol=0, atol=1e-15)


def _loop_attention(query, key, value, visible, scale):
    """Independent pair-by-pair restatement with math.exp (tiny cases only)."""

    q_tokens, q_heads, dim = query.shape
    group = q_heads // key.shape[1]
    out = np.zeros((q_tokens, q_heads, value.shape[2]))
    for i in range(q_tokens):
        for h in range(q_heads):
            kv = h // group
            scores = [sum(query[i, h, d] * key[j, kv, d] for d in range(dim)) * scale
                      for j in range(key.shape[0])]
            top = max(s for s, v in zip(scores, visible[i]) if v)
            weights = [math.exp(s - top) if v else 0.0 for s, v in zip(scores, visible[i])]
            total = sum(weights)
            for d in range(value.shape[2]):
                out[i, h, d] = sum(w * value[j, kv, d] for j, w in enumerate(weights)) / total
    return out


def test_oracle_matches_pairwise_loops_and_closed_forms():
    rng = np.random.default_rng(5)
    query = rng.standard_normal((3, 6, 4))
    key = rng.standard_normal((5, 2, 4))
    value = rng.standard_normal((5, 2, 4))
    visible = ao.logical_causal_mask(np.array([2, 3, 4]), np.arange(5))
    scale = 0.37
    assert np.allclose(ao.gqa_attention(query, key, value, visible, scale=scale),
                       _loop_attention(query, key, value, visible, scale), rtol=0, atol=1e-12)
    # One visible key: the output is that key's value row.
    only = np.zeros((3, 5), dtype=bool)
    only[:, 1] = True
    out = ao.gqa_attention(query, key, value, only)
    assert np.allclose(out[:, :3], value[1, 0][None, None, :]) and np.allclose(out[:, 3:], value[1, 1])
    # Zero queries: the mean of the visible values.
    out = ao.gqa_attention(np.zeros_like(query), key, value, visible)
    for i, p in enumerate([2, 3, 4]):
        assert np.allclose(out[i, 0], value[: p + 1, 0].mean(axis=0))
    # Invalid slots are invisible keys.
    pool_k, pool_v = rng.standard_normal((8, 2, 4)), rng.standard_normal((8, 2, 4))
    with_bad = ao.repair_attention(query[:2], pool_k, pool_v, [3, 9, 1, 0], 2, 4)
    visible = ao.logical_causal_mask(np.array([2, 3]), np.arange(4))
    visible[:, 1] = False
    safe = np.array([3, 0, 1, 0])
    assert np.allclose(with_bad, ao.gqa_attention(query[:2], pool_k[safe], pool_v[safe], visible))
    # ... whatever the row they alias holds.
    pool_k[0], pool_v[0] = np.inf, np.nan
    poisoned = ao.repair_attention(query[:2], pool_k, pool_v, [3, 9, 1, 11], 2, 4)
    assert np.isfinite(poisoned).all()
    assert np.allclose(poisoned, ao.repair_attention(query[:2], pool_k, pool_v, [3, -1, 1, 12], 2, 4))


def test_a_planted_head_mapping_mistake_fails_the_reference_case():
    query = np.zeros((1, 4, 2))
    key = np.zeros((1, 2, 2))
    value = np.array([[[10.0, 11.0], [20.0, 21.0]]])
    # h % num_kv_heads instead of h // group interleaves the heads.
    wrong = [value[0, h % 2, 0] for h in range(4)]
    assert wrong != ao.gqa_attention(query, key, value, np.ones((1, 1), dtype=bool))[0, :, 0].tolist()


def _plan(rows, q_heads=28, kv_heads=4, split=0):
    return _native.repair_attention_plan(np.asarray(rows, dtype=np.int64), q_heads, kv_heads, split)


@pytest.mark.parametrize("split,q_heads,kv_heads", [(0, 28, 4), (64, 28, 4), (512, 28, 4), (128, 8, 8),
                                                     (256, 8, 2)])
def test_plan_covers_every_query_and_key_range_once(split, q_heads, kv_heads):
    rng = np.random.default_rng(split + q_heads)
    rows, cursor = [], 0
    for _ in range(30):
        count = int(rng.integers(1, 40))
        start = int(rng.integers(0, 3000))
        rows.append((cursor, start, count, int(rng.integers(0, 3)) * 5000))  # three requests
        cursor += count
    items, combine, positions, info = _plan(rows, q_heads, kv_heads, split)
    T, H = _native.REPAIR_TILE_INTS, _native.REPAIR_ITEM_HEADER
    group = q_heads // kv_heads
    assert info.split_tokens % 64 == 0 and (split == 0 or info.split_tokens == split)
    # The positions table holds every query's logical position.
    position, request = np.zeros(cursor, np.int64), np.zeros(cursor, np.int64)
    for q_index, start, count, kv_off in rows:
        position[q_index : q_index + count] = np.arange(start, start + count)
        request[q_index : q_index + count] = kv_off
    assert info.num_queries == cursor and positions.tolist() == position.tolist()
    # Every item is a window of at most 16 (tile, query head) pairs, tile-major
    # from head pair_first of its first tile, ending in its last tile; every
    # pair entry: its tile's keys, a chunk of them, and its partial slot.
    covered, tiles = {}, set()
    for item in items.tolist():
        kv_off, kv_begin, kv_end, n_tiles, pair_first, pair_count = item[:H]
        assert 1 <= n_tiles <= 16 and kv_begin % 64 == 0 and kv_begin < kv_end
        assert 0 <= pair_first < group and 1 <= pair_count <= 16
        assert (pair_first + pair_count - 1) // group == n_tiles - 1
        furthest = 0
        for f in range(pair_first, pair_first + pair_count):
            t, head = divmod(f, group)
            q_index, low, q_count, partial, needed = item[H + T * t : H + T * (t + 1)]
            if q_count == 0:
                assert partial == -1
                continue
            assert 1 <= q_count <= 16
            queries = np.arange(q_index, q_index + q_count)
            assert (request[queries] == kv_off).all()          # one request per tile
            assert low == position[queries].min() and needed == position[queries].max() + 1
            furthest = max(furthest, needed)
            tiles.add((q_index, q_count, needed))
            covered.setdefault((q_index, q_count, head), []).append((kv_begin, min(kv_end, needed), partial, needed))
        assert kv_end <= furthest  # an item never loads keys past its last present tile's
    # Tiles partition the queries; consecutive rows of a request share tiles.
    seen = np.zeros(cursor, np.int64)
    for q_index, q_count, _ in tiles:
        seen[q_index : q_index + q_count] += 1
    assert (seen == 1).all()
    runs = []
    for q_index, start, count, kv_off in rows:
        if runs and runs[-1][0] == kv_off:
            runs[-1][1] += count
        else:
            runs.append([kv_off, count])
    run_tiles = [(n + 15) // 16 for _, n in runs]
    assert len(tiles) == sum(run_tiles)
    if q_heads == kv_heads:  # MHA: one head per KV head, windows of up to 16 tiles
        assert max(item[3] for item in items.tolist()) == min(16, max(run_tiles)) > 4
    # Windows are cut per run, at most 16 pairs each, and cover its pairs once.
    windows = {(item[H], item[4]): item[5] for item in items.tolist()}
    assert len(windows) >= sum((n * group + 15) // 16 for n in run_tiles)
    assert sum(windows.values()) == len(tiles) * group
    # Every (tile, query head) pair of every tile covers its keys once, in
    # chunks; its heads share the tile's partial slots.
    assert len(covered) == len(tiles) * group
    partials = set()
    combine_rows = [tuple(r) for r in combine.tolist()]
    slots_of = {}
    for (q_index, q_count, head), ranges in covered.items():
        ranges.sort()
        needed = ranges[0][3]
        assert ranges[0][0] == 0 and ranges[-1][1] == needed
        assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
        ids = [r[2] for r in ranges]
        assert slots_of.setdefault((q_index, q_count), ids) == ids
        if len(ranges) == 1:
            assert ids == [-1]
        else:
            assert ids == list(range(ids[0], ids[0] + len(ids)))
            partials.update(ids)
            assert (q_index, q_count, ids[0], len(ids)) in combine_rows
    assert len(partials) == info.workspace_items == combine[:, 3].sum()


def _windows(items):
    """(first query of the first tile, tiles, first head, pairs, keys) of each window."""
    H = _native.REPAIR_ITEM_HEADER
    spans = {}
    for item in items.tolist():
        key = (item[H], item[3], item[4], item[5])
        spans[key] = max(spans.get(key, 0), item[2])
    return sorted(key + (end,) for key, end in spans.items())


def test_plan_windows_cross_tiles_only_where_the_keys_match():
    # One 160-query span (10 tiles whose key ends are 16 apart), 7 query heads
    # per KV head: 70 pairs fit in five windows, four of 16 pairs crossing
    # tile boundaries, the short one on the tiles with the fewest keys.
    items, _, _, _ = _plan([(0, 5000, 160, 0)], 28, 4, 4096)
    assert [w[:4] for w in _windows(items)] == [(0, 1, 0, 6), (0, 4, 6, 16), (48, 3, 1, 16), (80, 3, 3, 16),
                                               (112, 3, 5, 16)]
    # Ten 16-query spans 1,000 positions apart: the same cuts.  A window's
    # cost is its furthest tile's keys, so the short window goes first (116
    # keys) and each later one ends where the tile-aligned pairs of tiles
    # (0-1, 2-3, ...) end: 2 + 49 + 80 + 112 + 143 key tiles against 18 + 49 +
    # 80 + 112 + 143.
    items, _, _, _ = _plan([(16 * i, 1000 * i + 100, 16, 0) for i in range(10)], 28, 4, 4096)
    assert _windows(items) == [(0, 1, 0, 6, 116), (0, 4, 6, 16, 3116), (48, 3, 1, 16, 5116),
                               (80, 3, 3, 16, 7116), (112, 3, 5, 16, 9116)]
    # 8 query heads per KV head: windows are whole pairs of tiles either way.
    items, _, _, _ = _plan([(0, 5000, 160, 0)], 64, 8, 4096)
    assert [w[:4] for w in _windows(items)] == [(32 * i, 2, 0, 16) for i in range(5)]


@pytest.mark.parametrize("seed", range(12))
def test_plan_windows_minimise_the_modelled_cost(seed):
    # Brute force over every cut of a short run's pairs into windows of at
    # most 16: the plan's windows cost the minimum of the planner's model
    # (key tiles of the window's furthest tile + 3 per window).
    rng = np.random.default_rng(seed)
    group = int(rng.choice([3, 5, 7]))
    n_tiles = 15 // group
    rows, cursor = [], 0
    for _ in range(n_tiles):
        start = int(rng.integers(0, 3000))
        rows.append((cursor, start, 16, 0))
        cursor += 16
    items, _, _, _ = _plan(rows, 4 * group, 4, 4096)
    needed = [start + 16 for _, start, _, _ in rows]
    pair_needed = [needed[p // group] for p in range(n_tiles * group)]

    def cost(cuts):
        bounds = [0, *cuts, len(pair_needed)]
        return sum(-(-max(pair_needed[a:b]) // 64) + 3 for a, b in zip(bounds, bounds[1:]))

    n = len(pair_needed)
    best = min(cost([c for c in range(1, n) if mask >> (c - 1) & 1]) for mask in range(1 << (n - 1))
               if all(b - a <= 16 for a, b in zip([0] + [c for c in range(1, n) if mask >> (c - 1) & 1],
                                                    [c for c in range(1, n) if mask >> (c - 1) & 1] + [n])))
    windows = _windows(items)
    assert sum(pairs for _, _, _, pairs, _ in windows) == n
    assert sum(-(-end // 64) + 3 for *_, end in windows) == best


def test_plan_packs_short_spans_of_one_request_into_tiles():
    # Four 8-query spans of one request: two full tiles; a span of another
    # request, or a gap in the query rows, starts a new tile.
    rows = [(0, 100, 8, 0), (8, 300, 8, 0), (16, 500, 8, 0), (24, 700, 8, 0), (32, 40, 8, 9000),
            (48, 60, 4, 9000)]
    items, combine, positions, info = _plan(rows, 28, 4, 4096)
    T, H = _native.REPAIR_TILE_INTS, _native.REPAIR_ITEM_HEADER
    tiles = sorted({tuple(item[H + T * t : H + T * (t + 1)]) for item in items.tolist() for t in range(item[3])
                    if item[H + T * t + 2]})
    assert tiles == [(0, 100, 16, -1, 308), (16, 500, 16, -1, 708), (32, 40, 8, -1, 48), (48, 60, 4, -1, 64)]
    assert positions[:16].tolist() == list(range(100, 108)) + list(range(300, 308))


def test_plan_rejects_bad_rows():
    with pytest.raises(_native.NativeCallError, match="row 0"):
        _plan([(0, 5, 0, 0)])
    with pytest.raises(_native.NativeCallError, match="row 1"):
        _plan([(0, 5, 3, 0), (3, -1, 3, 0)])
    with pytest.raises(_native.NativeCallError, match="multiple of 64"):
        _plan([(0, 5, 3, 0)], split=100)
    with pytest.raises(_native.NativeCallError, match="below 2"):
        _plan([(0, 5, 3, 0)], split=1 << 31)
    _plan([(0, 5, 3, 0)], split=7744)  # items longer than one slot-list fill run whole
    with pytest.raises(_native.NativeCallError) as error:
        _plan([(0, 5, 3, 0)], q_heads=30, kv_heads=4)  # not a multiple
    assert error.value.reason == "kv_head_layout_mismatch"
    _plan([(0, 5, 3, 0)], q_heads=71, kv_heads=1)  # any ratio, MQA included


def test_attention_entry_validates_before_any_launch():
    lib = _native.load_library()
    assert lib.ll_repair_attention_args_size() == ctypes.sizeof(_native.RepairAttentionArgs)
    assert lib.ll_repair_attention(None, None) == _native.LL_ERR_INVALID_ARGUMENT

    def args(**overrides):
        a = _native.RepairAttentionArgs()
        a.query, a.output, a.key_buffer, a.value_buffer = 0x1000, 0x2000, 0x3000, 0x4000
        a.num_queries, a.num_slots, a.num_q_heads, a.num_kv_heads, a.head_dim = 16, 64, 28, 4, 128
        a.kv_dtype = _native.DTYPE_BFLOAT16
        a.softmax_scale = 0.088
        a.kv_slots, a.kv_slots_dtype, a.kv_slots_len = 0x5000, _native.DTYPE_INT64, 64
        a.items, a.num_items = 0x6000, 1
        a.query_positions = 0x7000
        for name, value in overrides.items():
            setattr(a, name, value)
        return a

    for overrides, reason in [
        (dict(head_dim=96), "head_dimension_out_of_range"),
        (dict(head_dim=512), "head_dimension_out_of_range"),
        (dict(num_q_heads=30), "kv_head_layout_mismatch"),   # not a multiple of the KV heads
        (dict(num_q_heads=70000, num_kv_heads=1), "kv_head_layout_mismatch"),
        (dict(kv_dtype=_native.DTYPE_FLOAT32), "fp16_or_bf16_required"),
        (dict(kv_slots_dtype=_native.DTYPE_FLOAT32), "integer_token_maps_required"),
        (dict(query=None), "invalid_argument"),
        (dict(query_positions=None), "invalid_argument"),
        (dict(softmax_scale=float("nan")), "invalid_argument"),
        (dict(num_combine=1), "invalid_argument"),             # split items without a workspace
        (dict(query=0x1008), "invalid_argument"),              # misaligned
    ]:
        with pytest.raises(_native.NativeCallError) as error:
            _native.repair_attention(args(**overrides), 0)
        assert error.value.reason == reason, overrides
    _native.repair_attention(args(num_items=0), 0)  # nothing to do, no GPU touched


@pytest.mark.parametrize("seed", range(4))
def test_plan_filled_with_the_chosen_length_equals_a_searching_fill(seed):
    """The wrapper sizes the plan with the length search and fills it with the
    length that search chose; filling while searching again (both calls at 0)
    gives the same tables."""

    import ctypes

    rng = np.random.default_rng([9, seed])
    rows, cursor = [], 0
    for request in range(int(rng.integers(1, 5))):
        for _ in range(int(rng.integers(1, 60))):
            count = int(rng.integers(1, 33))
            rows.append((cursor, int(rng.integers(0, 30000)), count, request * 40000))
            cursor += count
    rows = np.asarray(rows, dtype=np.int64)
    items, combine, positions, info = _native.repair_attention_plan(rows, 28, 4, 0)
    lib = _native.load_library()
    again = _native.RepairPlanInfo()
    items2 = np.zeros_like(items)
    combine2 = np.zeros_like(combine)
    positions2 = np.zeros_like(positions)
    status = lib.ll_repair_attention_plan(
        rows.ctypes.data, rows.shape[0], 28, 4, 0, items2.ctypes.data if items2.size else None, items2.shape[0],
        combine2.ctypes.data if combine2.size else None, combine2.shape[0],
        positions2.ctypes.data if positions2.size else None, positions2.size, ctypes.byref(again))
    assert status == 0
    assert again.split_tokens == info.split_tokens and again.num_items == info.num_items
    assert np.array_equal(items, items2) and np.array_equal(combine, combine2)
    assert np.array_equal(positions, positions2)


def test_kept_plan_never_changes_results():
    """The planner keeps its last plan per thread; a plan asked again after
    other plans, with other heads or another chunk length, equals the one
    computed first, and a changed row is never served from the kept copy."""

    rng = np.random.default_rng(31)

    def random_rows(requests):
        rows, cursor = [], 0
        for request in range(requests):
            for _ in range(int(rng.integers(1, 40))):
                count = int(rng.integers(1, 33))
                rows.append((cursor, int(rng.integers(0, 20000)), count, request * 30000))
                cursor += count
        return np.asarray(rows, dtype=np.int64)

    a, b = random_rows(3), random_rows(2)
    first = _native.repair_attention_plan(a, 28, 4, 0)
    other = _native.repair_attention_plan(b, 28, 4, 0)
    assert not np.array_equal(first[0], other[0]) or first[0].shape != other[0].shape
    again = _native.repair_attention_plan(a, 28, 4, 0)
    for x, y in zip(first[:3], again[:3]):
        assert np.array_equal(x, y)
    assert first[3].split_tokens == again[3].split_tokens
    # Other heads, then an explicit length, on the same rows.
    grouped = _native.repair_attention_plan(a, 32, 4, 0)
    fresh_b = _native.repair_attention_plan(b, 28, 4, 0)
    grouped_again = _native.repair_attention_plan(a, 32, 4, 0)
    assert np.array_equal(grouped[0], grouped_again[0]) and np.array_equal(fresh_b[0], other[0])
    explicit = _native.repair_attention_plan(a, 28, 4, 1024)
    assert explicit[3].split_tokens == 1024
    _native.repair_attention_plan(b, 28, 4, 0)
    explicit_again = _native.repair_attention_plan(a, 28, 4, 1024)
    assert np.array_equal(explicit[0], explicit_again[0]) and np.array_equal(explicit[1], explicit_again[1])
    # One changed row right after the plan it would otherwise match.
    changed = a.copy()
    changed[-1, 1] += 1
    plan_changed = _native.repair_attention_plan(changed, 28, 4, 0)
    assert not np.array_equal(plan_changed[2], first[2])
    assert plan_changed[2][-1] == first[2][-1] + 1


def test_plan_span_checks_report_the_first_failing_span():
    """The checks of build_explicit_causal_pattern (flashinfer_sparse_repair.py:
    1217-1238) in span order: the first span that fails decides the message,
    its tensor's checks before its range checks."""

    import torch

    from legolink_amd.repair_attention import RepairAttentionPlan, SparseRepairAttentionError

    good = torch.arange(10, dtype=torch.int64)
    rank2 = torch.arange(10, dtype=torch.int64).view(2, 5)
    floats = torch.arange(10, dtype=torch.float32)
    meta = torch.empty(10, dtype=torch.int64, device="meta")
    cases = [
        ([(good, 0, 4), (floats, 0, 2)], "int32 or int64"),
        ([(good, 3, 3), (rank2, 0, 1)], "invalid repair range"),
        ([(rank2, 0, 1), (good, 3, 3)], "rank 1"),
        ([(good, 0, 4), (good, 5, 11)], "shorter than repair_end"),
        ([(good, 5, 11), (good, -1, 2)], "shorter than repair_end"),
        ([(good, 0, 4), (good, -1, 2), (floats, 0, 1)], "invalid repair range"),
        ([(good, 0, 4), (meta, 0, 2)], "share one device"),
    ]
    for spans, message in cases:
        with pytest.raises(SparseRepairAttentionError, match=message):
            RepairAttentionPlan(spans, num_q_heads=8, num_kv_heads=2, head_dim=64, pool_size=100)
    with pytest.raises(SparseRepairAttentionError, match="no repair spans"):
        RepairAttentionPlan([], num_q_heads=8, num_kv_heads=2, head_dim=64)
    # Slots outside the pool, up to the spans' largest end only.
    slots = torch.tensor([3, 7, 99, 100, -1], dtype=torch.int64)
    RepairAttentionPlan([(slots, 1, 3)], num_q_heads=8, num_kv_heads=2, head_dim=64, pool_size=100)
    for end, size in ((4, 100), (3, 99)):
        with pytest.raises(SparseRepairAttentionError, match="invalid KV slots"):
            RepairAttentionPlan([(slots, 1, end)], num_q_heads=8, num_kv_heads=2, head_dim=64, pool_size=size)
    RepairAttentionPlan([(slots, 0, 5)], num_q_heads=8, num_kv_heads=2, head_dim=64, validate=False,
                        pool_size=100)


def test_plan_rows_and_slot_table_of_shared_and_mixed_tensors():
    import torch

    from legolink_amd.repair_attention import RepairAttentionPlan

    a = torch.arange(100, 140, dtype=torch.int64)
    b = torch.arange(500, 520, dtype=torch.int32)
    spans = [(a, 4, 9), (b, 2, 3), (a, 20, 36), (b, 10, 20), (a, 39, 40)]
    plan = RepairAttentionPlan(spans, num_q_heads=28, num_kv_heads=4, head_dim=128, pool_size=1000)
    # One table: a's slots, then b's (as int64); rows (query index, start, count, table offset).
    assert plan.kv_slots.dtype == torch.int64
    assert plan.kv_slots.tolist() == list(range(100, 140)) + list(range(500, 520))
    expected, cursor = [], 0
    for tensor, start, end in spans:
        expected.append([cursor, start, end - start, 0 if tensor is a else 40])
        cursor += end - start
    assert plan.rows.tolist() == expected and plan.num_queries == cursor
    # Bounds given as numpy integers or 0-dim tensors read the same.
    odd = [(a, np.int64(4), torch.tensor(9)), (b, 2, np.int32(3))]
    plan2 = RepairAttentionPlan(odd, num_q_heads=28, num_kv_heads=4, head_dim=128)
    assert plan2.rows.tolist() == [[0, 4, 5, 0], [5, 2, 1, 40]]
    pairs = sum((e - s) * (s + e + 1) // 2 for _, s, e in spans)
    assert plan.algorithmic_flops == 4 * 128 * 28 * pairs
