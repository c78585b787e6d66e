"""Token maps of a link, built on the device from the plan's runs.

The reference materialises a link's maps on the host, block by block
(patched_sglang_files/python/sglang/srt/pic_runtime.py:4905-5003): the
request's destination slots ``[start, end)`` of each block, its compile-time
positions ``arange(n)``, its global positions ``start + arange(n)``, then a
``torch.cat`` of every map and, with boundary-repair awareness, a uint8 mask
of the ``imp_indices`` rows built on the host and copied over.

Here the host only cuts the plan into runs, vectorised over blocks: a run is
a stretch of one block holding at most one contiguous run of repair rows.
One call of ``ll_kv_build_link_maps`` then writes every map of the link, in
plan order, per source set (0: pool slots, 1: snapshot arena), with repair
rows either left out (compacted) or flagged in a mask, and the destination
slots of the repair rows for the write-back.  The output equals the
reference's concatenation restricted to each set, in the same order.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native

_FIELD = {name: index for index, name in enumerate(_native.SEGMENT_FIELDS)}


@dataclass
class BlockTable:
    """A link's blocks in plan order (one entry per block)."""

    starts: np.ndarray        # int64 [B] request position of the block's first token
    counts: np.ndarray        # int64 [B] tokens
    source_ptrs: np.ndarray   # int64 [B] device address of the block's int64 source slots
    local_ptrs: np.ndarray    # int64 [B] device address of int64 local positions, 0: affine
    local_starts: np.ndarray  # int64 [B] local position of token 0 (affine blocks)
    sets: np.ndarray          # int64 [B] 0: pool slots, 1: snapshot arena
    destination_bases: Optional[np.ndarray] = None  # int64 [B] offset of the block's request
                                                     # in the destination slots (None: 0)

    @property
    def destination_starts(self) -> np.ndarray:
        """Index of every block's first destination slot."""

        return self.starts if self.destination_bases is None else self.starts + self.destination_bases

    @property
    def offsets(self) -> np.ndarray:
        """Concatenation offset of every block's first token."""

        return np.concatenate(([0], np.cumsum(self.counts)[:-1])).astype(np.int64)

    @property
    def token_count(self) -> int:
        return int(self.counts.sum())


@dataclass
class SegmentPlan:
    table: np.ndarray           # int64 [S, 11]: ll_link_segment records
    map_counts: tuple[int, int]  # map entries of set 0 and set 1
    set_repair_rows: tuple[int, int]  # repair rows whose tokens belong to each set
    repair_count: int           # repair rows recorded (write-back order = plan order)
    repair_offsets: np.ndarray  # int64 [R] concatenation offsets of the repair rows
    block_entries: np.ndarray   # int64 [B] map entries each block contributes
    set_prefix: tuple[int, int]  # identity tokens at the head of each set's maps
    segment_blocks: Optional[np.ndarray] = None  # int64 [S] block of every run

    def run_entries(self, compact: bool) -> np.ndarray:
        """Map entries of every run (its tokens, less its repair rows when compacted)."""

        table = self.table
        entries = table[:, _FIELD["token_count"]]
        if compact:
            entries = entries - (table[:, _FIELD["repair_end"]] - table[:, _FIELD["repair_begin"]])
        return entries


def exclusive_offsets(sizes: np.ndarray) -> np.ndarray:
    """int64 offset of every entry in the concatenation of ``sizes``."""

    out = np.zeros(sizes.shape[0], dtype=np.int64)
    if sizes.shape[0] > 1:
        np.cumsum(sizes[:-1], out=out[1:])
    return out


def repair_rows_in_blocks(blocks: BlockTable, repair_positions: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(block index, offset in block) of every repair position inside a block,
    sorted in plan order; positions outside every block are dropped
    (pic_runtime.py:4981-5003 keeps ``start <= position < end`` only).

    Positions are destination indices: the request position plus the
    request's offset in the destination slots (0 for a single request)."""

    positions = _sorted_unique(np.asarray(repair_positions, dtype=np.int64).reshape(-1))
    if positions.size == 0 or blocks.counts.size == 0:
        empty = np.zeros(0, dtype=np.int64)
        return empty, empty
    starts = blocks.destination_starts
    in_position_order = blocks.counts.size == 1 or bool(np.all(starts[1:] > starts[:-1]))
    order = None if in_position_order else np.argsort(starts, kind="stable")
    sorted_starts = starts if order is None else starts[order]
    slot = np.searchsorted(sorted_starts, positions, side="right") - 1
    inside = slot >= 0
    slot_c = np.where(inside, slot, 0)
    block = slot_c if order is None else order[slot_c]
    inside &= positions < starts[block] + blocks.counts[block]
    block = block[inside]
    offset = positions[inside] - starts[block]
    if order is None:
        # Blocks in position order: position order is plan order already.
        return block, offset
    concat = blocks.offsets[block] + offset
    ordering = np.argsort(concat, kind="stable")
    return block[ordering], offset[ordering]


def _sorted_unique(values: np.ndarray) -> np.ndarray:
    if values.size > 1 and not bool(np.all(values[1:] > values[:-1])):
        return np.unique(values)
    return values


_BLOCK_FIELD = {name: index for index, name in enumerate(_native.BLOCK_FIELDS)}


def plan_segments(blocks: BlockTable, repair_positions: np.ndarray, *, compact: bool,
                  leading_blocks: Optional[np.ndarray] = None) -> SegmentPlan:
    """Cut the blocks into runs with at most one contiguous repair run each
    (``ll_plan_link_runs``, host C++).

    ``repair_positions`` are destination indices (request positions for one
    request; sorted or not, duplicates allowed); only those inside blocks
    count.  With ``compact`` the repair rows take no map entry; otherwise
    they are flagged in the set's mask.  Runs of ``leading_blocks`` (the
    identity blocks: no token needs a remap) take the first map entries of
    their set, in plan order, so they form the set's identity prefix; the
    other runs follow in plan order.  The runs themselves, and so the order
    of the repair rows, stay in plan order.
    """

    count_blocks = int(blocks.counts.size)
    records = np.empty((count_blocks, len(_BLOCK_FIELD)), dtype=np.int64)
    records[:, _BLOCK_FIELD["source_slots"]] = blocks.source_ptrs
    records[:, _BLOCK_FIELD["local_positions"]] = blocks.local_ptrs
    records[:, _BLOCK_FIELD["token_count"]] = blocks.counts
    records[:, _BLOCK_FIELD["start_token"]] = blocks.starts
    records[:, _BLOCK_FIELD["destination_base"]] = (0 if blocks.destination_bases is None
                                                    else blocks.destination_bases)
    records[:, _BLOCK_FIELD["local_start"]] = blocks.local_starts
    records[:, _BLOCK_FIELD["map_set"]] = blocks.sets
    records[:, _BLOCK_FIELD["leading"]] = (0 if leading_blocks is None
                                           else np.asarray(leading_blocks, dtype=np.int64))
    table, segment_blocks, repair_offsets, info = _native.plan_link_runs(
        records, np.asarray(repair_positions, dtype=np.int64).reshape(-1), compact)
    entries = table[:, _FIELD["token_count"]] - (
        table[:, _FIELD["repair_end"]] - table[:, _FIELD["repair_begin"]] if compact else 0)
    return SegmentPlan(
        table=table,
        map_counts=(int(info.map_count[0]), int(info.map_count[1])),
        set_repair_rows=(int(info.set_repair_rows[0]), int(info.set_repair_rows[1])),
        repair_count=int(info.repair_count),
        repair_offsets=repair_offsets,
        block_entries=np.bincount(segment_blocks, weights=entries, minlength=count_blocks).astype(np.int64),
        set_prefix=(int(info.set_prefix[0]), int(info.set_prefix[1])),
        segment_blocks=segment_blocks,
    )


@dataclass
class DeviceMaps:
    """Output of the map builder: per set an int64 ``[4, n]`` map tensor (rows:
    source slots, destination slots, local positions, global positions) and
    an optional uint8 mask; the destination slots of the repair rows."""

    maps: list[Optional[torch.Tensor]]
    masks: list[Optional[torch.Tensor]]
    repair_destination_slots: torch.Tensor
    run_table: Optional[torch.Tensor] = None  # the device copy of the runs the builder read


def set_entry_flags(plan: SegmentPlan, source_set: int, run_flags: np.ndarray, *, compact: bool) -> np.ndarray:
    """A per-run flag spread over the map entries of one set: uint8 ``[n]`` with
    entry ``o`` holding the flag of the run that writes map entry ``o``."""

    table = plan.table
    pick = table[:, _FIELD["map_set"]] == source_set
    offsets = table[pick, _FIELD["map_offset"]]
    entries = plan.run_entries(compact)[pick]
    order = np.argsort(offsets, kind="stable")
    flags = np.repeat(np.asarray(run_flags, dtype=np.uint8)[pick][order], entries[order])
    if flags.size != plan.map_counts[source_set]:
        raise AssertionError("the runs of a set do not tile its map entries")
    return flags


# Above this many runs the map builder reads them from a device copy of the
# run table (one launch) instead of its kernel arguments (56 runs a launch).
DEVICE_TABLE_RUNS = 56


def build_device_maps(plan: SegmentPlan, destination_slots: torch.Tensor, *, compact: bool,
                      stream: torch.cuda.Stream | None = None) -> DeviceMaps:
    """Enqueue the map builder on ``stream`` (default: the current stream)."""

    device = destination_slots.device
    if not destination_slots.is_cuda:
        # The reason string of the operator's eligibility check for host tensors.
        raise RuntimeError("HIP LegoLink fusion is unavailable: cuda_tensors_required")
    if destination_slots.dtype not in (torch.int32, torch.int64) or not destination_slots.is_contiguous():
        raise ValueError("destination slots must be a contiguous int32 or int64 tensor")
    maps: list[Optional[torch.Tensor]] = []
    masks: list[Optional[torch.Tensor]] = []
    for s in (0, 1):
        n = plan.map_counts[s]
        maps.append(torch.empty((4, n), dtype=torch.int64, device=device) if n else None)
        masks.append(torch.empty(n, dtype=torch.uint8, device=device) if n and not compact else None)
    repair = torch.empty(plan.repair_count, dtype=torch.int64, device=device)
    args = _native.LinkMapsArgs()
    table = np.ascontiguousarray(plan.table)
    args.num_segments = int(table.shape[0])
    args.segments = table.ctypes.data if table.size else None
    args.destination_slots = destination_slots.data_ptr()
    args.destination_slots_dtype = (_native.DTYPE_INT64 if destination_slots.dtype == torch.int64
                                    else _native.DTYPE_INT32)
    args.num_destination_slots = int(destination_slots.numel())
    for s in (0, 1):
        args.maps[s] = maps[s].data_ptr() if maps[s] is not None else None
        args.map_capacity[s] = plan.map_counts[s]
        args.repair_mask[s] = masks[s].data_ptr() if masks[s] is not None else None
    args.repair_destination_slots = repair.data_ptr() if plan.repair_count else None
    args.repair_capacity = plan.repair_count
    if stream is None:
        stream = torch.cuda.current_stream(device)
    device_table = None
    if args.num_segments > DEVICE_TABLE_RUNS:
        # Many runs: one copy of the run table to the device and one launch,
        # where the kernel arguments would take a launch per 56 runs.  The
        # copy is ordered before the builder on its stream.
        with torch.cuda.stream(stream):
            device_table = torch.from_numpy(table).pin_memory().to(device, non_blocking=True)
        args.device_segments = device_table.data_ptr()
    _native.kv_build_link_maps(args, stream.cuda_stream)
    return DeviceMaps(maps=maps, masks=masks, repair_destination_slots=repair, run_table=device_table)


def order_link_maps(maps: torch.Tensor, mask: Optional[torch.Tensor], *, key_row: int, prefix: int,
                    num_slots: int, workspace: torch.Tensor,
                    stream: torch.cuda.Stream | None = None) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """A map set's entries [prefix, n) ordered by the slots of map row
    ``key_row`` (0: source slots, 1: destination slots), in buckets of 2^shift
    slots (16,384 buckets over the ``num_slots`` rows of the pool those slots
    index; one slot per bucket up to 16,384 rows); entries [0, prefix) stay
    first and in place, and the mask follows its entries.  ``workspace`` is a
    zeroed uint8 device tensor of ``_native.ORDER_WORKSPACE_BYTES`` that calls
    on one stream may share (``ll_order_link_maps``)."""

    if key_row not in (0, 1):
        raise ValueError("key_row must be 0 (source slots) or 1 (destination slots)")
    n = int(maps.shape[1])
    out = torch.empty_like(maps)
    out_mask = None if mask is None else torch.empty_like(mask)
    args = _native.OrderMapsArgs()
    args.maps = maps.data_ptr()
    args.mask = None if mask is None else mask.data_ptr()
    args.capacity = n
    args.count = n
    args.prefix = int(prefix)
    args.num_slots = int(num_slots)
    args.out_maps = out.data_ptr()
    args.out_mask = None if out_mask is None else out_mask.data_ptr()
    args.workspace = workspace.data_ptr()
    args.workspace_bytes = int(workspace.numel())
    args.key_row = int(key_row)
    if stream is None:
        stream = torch.cuda.current_stream(maps.device)
    _native.order_link_maps(args, stream.cuda_stream)
    return out, out_mask


def order_by_destination(maps: torch.Tensor, mask: Optional[torch.Tensor], *, prefix: int, num_slots: int,
                         workspace: torch.Tensor,
                         stream: torch.cuda.Stream | None = None) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """``order_link_maps`` by destination slot."""

    return order_link_maps(maps, mask, key_row=1, prefix=prefix, num_slots=num_slots, workspace=workspace,
                           stream=stream)


def block_table(starts: Sequence[int], counts: Sequence[int], source_ptrs: Sequence[int],
                local_ptrs: Sequence[int], local_starts: Sequence[int], sets: Sequence[int],
                destination_bases: Optional[Sequence[int]] = None) -> BlockTable:
    as64 = lambda values: np.asarray(values, dtype=np.int64).reshape(-1)
    return BlockTable(starts=as64(starts), counts=as64(counts), source_ptrs=as64(source_ptrs),
                      local_ptrs=as64(local_ptrs), local_starts=as64(local_starts), sets=as64(sets),
                      destination_bases=None if destination_bases is None else as64(destination_bases))


def concatenate_tables(tables: Sequence[BlockTable], bases: Sequence[int]) -> BlockTable:
    """Blocks of several requests, request after request; request r's
    destination slots start at ``bases[r]`` in the concatenated slots."""

    counts = [t.counts.size for t in tables]
    own = [t.destination_bases if t.destination_bases is not None else np.zeros(n, dtype=np.int64)
           for t, n in zip(tables, counts)]
    return BlockTable(
        starts=np.concatenate([t.starts for t in tables]),
        counts=np.concatenate([t.counts for t in tables]),
        source_ptrs=np.concatenate([t.source_ptrs for t in tables]),
        local_ptrs=np.concatenate([t.local_ptrs for t in tables]),
        local_starts=np.concatenate([t.local_starts for t in tables]),
        sets=np.concatenate([t.sets for t in tables]),
        destination_bases=np.concatenate([o + int(b) for o, b in zip(own, bases)]).astype(np.int64),
    )
