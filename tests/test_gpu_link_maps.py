"""GPU parity of the map builder (ll_kv_build_link_maps) against the oracle's
maps: bit-exact integers on random plans, both repair-row forms, both source
sets, consecutive and explicit compile-time positions, int32 and int64
request slots, more runs than one launch takes, and runs longer than one
workgroup row."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from legolink_amd import link_maps
from oracle import link_maps_oracle as lmo
from tests.gpu_helpers import report
from tests.test_link_maps import _random_plan

pytestmark = pytest.mark.gpu


def _device_table(blocks, device):
    keep = []
    starts, counts, sources, locals_, local_starts, sets = [], [], [], [], [], []
    for block in blocks:
        slots = torch.from_numpy(np.asarray(block["source_slots"], dtype=np.int64)).to(device)
        local = np.asarray(block["local_positions"], dtype=np.int64)
        n = local.size
        keep.append(slots)
        starts.append(block["start"])
        counts.append(n)
        sources.append(slots.data_ptr())
        if np.array_equal(local, local[0] + np.arange(n)):
            locals_.append(0)
            local_starts.append(int(local[0]))
        else:
            local_t = torch.from_numpy(local).to(device)
            keep.append(local_t)
            locals_.append(local_t.data_ptr())
            local_starts.append(0)
        sets.append(block["set"])
    return link_maps.block_table(starts, counts, sources, locals_, local_starts, sets), keep


CASES = [
    # name, seed, blocks, max block length, compact, request slot dtype
    ("small_compact", 1, None, 40, True, torch.int64),
    ("small_masked", 2, None, 40, False, torch.int64),
    ("int32_request_slots", 3, None, 40, True, torch.int32),
    ("many_runs_several_launches", 4, 150, 30, True, torch.int64),
    ("many_runs_masked", 5, 150, 30, False, torch.int32),
    ("long_blocks_several_rows", 6, 5, 5000, True, torch.int64),
]


@pytest.mark.parametrize("run_table", ["kernel_arguments", "device_table"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_device_maps_match_oracle(gpu_device, case, run_table, monkeypatch):
    """Both ways the runs reach the builder: in kernel arguments (56 runs a
    launch) and from a device copy of the run table (one launch)."""

    monkeypatch.setattr(link_maps, "DEVICE_TABLE_RUNS", 0 if run_table == "device_table" else 1 << 30)
    name, seed, count, max_len, compact, slot_dtype = case
    name = f"{name}/{run_table}"
    rng = np.random.default_rng(seed)
    for trial in range(4):
        blocks, request_slots, imp = _random_plan(rng, blocks=count, max_len=max_len)
        table, keep = _device_table(blocks, gpu_device)
        plan = link_maps.plan_segments(table, np.asarray(imp, dtype=np.int64), compact=compact)
        report(f"case {name} trial {trial}: {len(blocks)} blocks, {plan.table.shape[0]} runs, "
               f"maps {plan.map_counts}, repair rows {plan.repair_count}")
        slots_device = torch.from_numpy(request_slots).to(slot_dtype).to(gpu_device)
        built = link_maps.build_device_maps(plan, slots_device, compact=compact)
        assert (built.run_table is not None) == (run_table == "device_table")
        torch.cuda.synchronize(gpu_device)
        expected = lmo.device_maps(blocks, request_slots, imp, compact=compact)
        assert np.array_equal(built.repair_destination_slots.cpu().numpy(),
                              expected["repair_destination_slots"])
        for s in (0, 1):
            if expected[f"maps{s}"] is None:
                assert built.maps[s] is None
                continue
            assert np.array_equal(built.maps[s].cpu().numpy(), expected[f"maps{s}"]), (name, trial, s)
            if compact:
                assert built.masks[s] is None
            else:
                assert np.array_equal(built.masks[s].cpu().numpy(), expected[f"mask{s}"])
        del keep


def test_batched_device_maps_match_oracle(gpu_device):
    rng = np.random.default_rng(41)
    for trial in range(3):
        compact = trial != 1
        requests, tables, keep, bases, leading, repairs = [], [], [], [], [], []
        base = 0
        for _ in range(int(rng.integers(3, 7))):
            blocks, slots, imp = _random_plan(rng, max_len=60)
            table, kept = _device_table(blocks, gpu_device)
            requests.append((blocks, slots, imp))
            tables.append(table)
            keep.extend(kept)
            bases.append(base)
            lead = np.zeros(len(blocks), dtype=bool)
            lead[0] = lmo.concatenated_maps(blocks, slots, imp)["prefix_token_count"] > 0
            leading.append(lead)
            repairs.append(np.asarray(imp, dtype=np.int64) + base)
            base += slots.size
        plan = link_maps.plan_segments(link_maps.concatenate_tables(tables, bases), np.concatenate(repairs),
                                       compact=compact, leading_blocks=np.concatenate(leading))
        report(f"batched maps trial {trial}: {len(requests)} requests, {plan.table.shape[0]} runs")
        all_slots = torch.from_numpy(np.concatenate([s for _, s, _ in requests])).to(gpu_device)
        built = link_maps.build_device_maps(plan, all_slots, compact=compact)
        torch.cuda.synchronize(gpu_device)
        expected = lmo.batched_device_maps(requests, compact=compact)
        assert np.array_equal(built.repair_destination_slots.cpu().numpy(),
                              expected["repair_destination_slots"])
        for s in (0, 1):
            assert plan.set_prefix[s] == expected[f"prefix{s}"]
            if expected[f"maps{s}"] is None:
                assert built.maps[s] is None
                continue
            assert np.array_equal(built.maps[s].cpu().numpy(), expected[f"maps{s}"])
            if not compact:
                assert np.array_equal(built.masks[s].cpu().numpy(), expected[f"mask{s}"])
        del keep


def test_device_table_runs_are_checked_again_on_the_device(gpu_device):
    """A device run table that differs from the host's (map offsets past the
    capacity, a destination range past the request, a repair range past its
    capacity) loses those runs; the others are built.  The buffers are
    allocated larger than the sizes passed, so a read or write past one would
    still land inside them, and the test checks that no write did."""

    from legolink_amd import _native

    rng = np.random.default_rng(11)
    blocks, request_slots, imp = _random_plan(rng, blocks=12, max_len=30)
    table, keep = _device_table(blocks, gpu_device)
    plan = link_maps.plan_segments(table, np.asarray(imp, dtype=np.int64), compact=True)
    runs = np.ascontiguousarray(plan.table).copy()
    field = {name: i for i, name in enumerate(_native.SEGMENT_FIELDS)}
    guard = 4096
    slot_buffer = torch.zeros(request_slots.size + guard, dtype=torch.int64, device=gpu_device)
    slots = slot_buffer[: request_slots.size]
    slots.copy_(torch.from_numpy(request_slots))
    capacity = [plan.map_counts[0], plan.map_counts[1]]
    maps = [torch.full((4 * c + guard,), -7, dtype=torch.int64, device=gpu_device) for c in capacity]
    repair = torch.full((plan.repair_count + guard,), -7, dtype=torch.int64, device=gpu_device)
    corrupt = runs.copy()
    nonempty = np.flatnonzero(corrupt[:, field["token_count"]] > 0)
    bad = nonempty[:3]
    corrupt[bad[0], field["map_offset"]] = capacity[int(corrupt[bad[0], field["map_set"]])]
    corrupt[bad[1], field["destination_start"]] = request_slots.size
    with_repair = [k for k in nonempty if corrupt[k, field["repair_end"]] > corrupt[k, field["repair_begin"]]]
    if with_repair:
        corrupt[with_repair[-1], field["repair_offset"]] = plan.repair_count
    device_runs = torch.from_numpy(corrupt).to(gpu_device)
    args = _native.LinkMapsArgs()
    args.num_segments = runs.shape[0]
    args.segments = runs.ctypes.data
    args.destination_slots = slots.data_ptr()
    args.destination_slots_dtype = _native.DTYPE_INT64
    args.num_destination_slots = slots.numel()
    for s in (0, 1):
        args.maps[s] = maps[s].data_ptr() if capacity[s] else None
        args.map_capacity[s] = capacity[s]
    args.repair_destination_slots = repair.data_ptr() if plan.repair_count else None
    args.repair_capacity = plan.repair_count
    args.device_segments = device_runs.data_ptr()
    report(f"device table re-check: {runs.shape[0]} runs, corrupted {bad.tolist()}")
    _native.kv_build_link_maps(args, torch.cuda.current_stream(gpu_device).cuda_stream)
    torch.cuda.synchronize(gpu_device)
    for s in (0, 1):
        assert (maps[s][4 * capacity[s]:] == -7).all(), "a write past the map capacity"
    assert (repair[plan.repair_count:] == -7).all(), "a write past the repair capacity"
    # The runs left intact are built as the host table says.
    expected = link_maps.build_device_maps(plan, slots, compact=True)
    torch.cuda.synchronize(gpu_device)
    skipped = set(bad[:2].tolist()) | ({with_repair[-1]} if with_repair else set())
    for k in range(runs.shape[0]):
        s = int(runs[k, field["map_set"]])
        count = int(runs[k, field["token_count"]])
        if k in skipped or count == 0 or expected.maps[s] is None:
            continue
        rb, re = int(runs[k, field["repair_begin"]]), int(runs[k, field["repair_end"]])
        begin = int(runs[k, field["map_offset"]])
        entries = count - (re - rb)
        got = maps[s][: 4 * capacity[s]].view(4, capacity[s])[:, begin : begin + entries]
        assert torch.equal(got, expected.maps[s][:, begin : begin + entries]), k
    del keep
