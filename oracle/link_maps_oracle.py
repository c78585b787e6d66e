"""CPU oracle of a link's token maps.

TEST INFRASTRUCTURE ONLY: only tests/ may import this module, to check the
device map builder.  The product path never calls it.

Restates, block by block in plan order, the map construction of
``_copy_linked_kv_batched_blocks``
(patched_sglang_files/python/sglang/srt/pic_runtime.py:4905-5013):

* destination slots = ``destination_slots[start:end]``          (:4933)
* local positions   = the block's compile-time positions        (:4934-4936 use arange(n))
* global positions  = ``start + arange(n)``                      (:4951)
* source slots      = the block's registered slots               (:4970-4974)
* repair offsets    = ``concatenated_offset + position - start`` for every
  unique ``imp_indices`` position with ``start <= position < end`` (:4981-4990)
* identity prefix   = block 0's token count when none of its tokens needs a
  remap, else 0                                                  (:5005-5013)

and then the two forms the device builder emits: the maps split by source
(pool slots or snapshot arena, pic_runtime.py:5553-5567 links clone blocks
from their snapshot), each in plan order, with the repair rows either removed
(compacted) or kept and flagged in a uint8 mask; plus the destination slots
of the repair rows in plan order (the rows the write-back fills).  For a
batch of requests linked as one (no counterpart in the reference, which links
request by request), each request's identity prefix moves to the head of its
set so that it is still the leading, unrotated run.
"""

from __future__ import annotations

from typing import Any, Sequence

import numpy as np


def concatenated_maps(blocks: Sequence[dict[str, Any]], request_slots: np.ndarray,
                      imp_indices: Sequence[int]) -> dict[str, Any]:
    """Plan-order maps of the whole link.

    ``blocks``: dicts with ``start``, ``source_slots`` (int64 [n]),
    ``local_positions`` (int64 [n]) and ``set`` (0 pool, 1 arena).
    """

    request_slots = np.asarray(request_slots, dtype=np.int64)
    unique_repairs = sorted(set(int(p) for p in imp_indices))
    src, dst, local, glob, sets, repair_offsets = [], [], [], [], [], []
    offset = 0
    for block in blocks:
        start = int(block["start"])
        slots = np.asarray(block["source_slots"], dtype=np.int64)
        n = int(slots.size)
        end = start + n
        src.append(slots)
        dst.append(request_slots[start:end])
        local.append(np.asarray(block["local_positions"], dtype=np.int64))
        glob.append(np.arange(start, end, dtype=np.int64))
        sets.append(np.full(n, int(block["set"]), dtype=np.int64))
        repair_offsets.extend(offset + p - start for p in unique_repairs if start <= p < end)
        offset += n
    first_local = np.asarray(blocks[0]["local_positions"], dtype=np.int64)
    first_start = int(blocks[0]["start"])
    identity = np.array_equal(first_local, np.arange(first_start, first_start + first_local.size))
    return {
        "source_slots": np.concatenate(src),
        "destination_slots": np.concatenate(dst),
        "local_positions": np.concatenate(local),
        "global_positions": np.concatenate(glob),
        "sets": np.concatenate(sets),
        "repair_offsets": np.asarray(repair_offsets, dtype=np.int64),
        "prefix_token_count": int(first_local.size) if identity else 0,
    }


def batched_device_maps(requests: Sequence[tuple[Sequence[dict[str, Any]], np.ndarray, Sequence[int]]],
                        *, compact: bool) -> dict[str, Any]:
    """What the map builder must write for several requests linked as one:
    each request's maps as above; per set, the requests' identity-prefix
    tokens first (request after request), then their other tokens (request
    after request), each in plan order; the repair rows' destination slots
    request after request."""

    per = [concatenated_maps(blocks, slots, imp) for blocks, slots, imp in requests]
    out: dict[str, Any] = {
        "repair_destination_slots": np.concatenate(
            [m["destination_slots"][m["repair_offsets"]] for m in per]).astype(np.int64),
    }
    names = ("source_slots", "destination_slots", "local_positions", "global_positions")
    for s in (0, 1):
        heads, tails, head_masks, tail_masks = [], [], [], []
        for m in per:
            n = m["source_slots"].size
            is_repair = np.zeros(n, dtype=bool)
            is_repair[m["repair_offsets"]] = True
            in_prefix = np.arange(n) < m["prefix_token_count"]
            members = m["sets"] == s
            selected = members & ~is_repair if compact else members
            stacked = np.stack([m[name] for name in names])
            head = in_prefix & selected
            tail = ~in_prefix & selected
            heads.append(stacked[:, head])
            tails.append(stacked[:, tail])
            head_masks.append(is_repair[head])
            tail_masks.append(is_repair[tail])
        maps = np.concatenate(heads + tails, axis=1)
        out[f"maps{s}"] = maps if maps.shape[1] else None
        out[f"mask{s}"] = (np.concatenate(head_masks + tail_masks).astype(np.uint8)
                           if not compact and maps.shape[1] else None)
        out[f"prefix{s}"] = int(sum(h.shape[1] for h in heads))
    return out


def device_maps(blocks: Sequence[dict[str, Any]], request_slots: np.ndarray,
                imp_indices: Sequence[int], *, compact: bool) -> dict[str, Any]:
    """What the map builder must write: per set ``maps`` (int64 [4, n]: source,
    destination, local, global), ``mask`` (uint8 [n], or None when compacted)
    and ``prefix`` (identity tokens at the head of the set's maps); and
    ``repair_destination_slots`` in plan order."""

    whole = concatenated_maps(blocks, request_slots, imp_indices)
    token_count = whole["source_slots"].size
    is_repair = np.zeros(token_count, dtype=bool)
    is_repair[whole["repair_offsets"]] = True
    in_prefix = np.arange(token_count) < whole["prefix_token_count"]
    out: dict[str, Any] = {
        "repair_destination_slots": whole["destination_slots"][whole["repair_offsets"]],
        "repair_offsets": whole["repair_offsets"],
        "prefix_token_count": whole["prefix_token_count"],
    }
    for s in (0, 1):
        members = whole["sets"] == s
        selected = members & ~is_repair if compact else members
        maps = np.stack([whole[name][selected] for name in
                         ("source_slots", "destination_slots", "local_positions", "global_positions")])
        out[f"maps{s}"] = maps if maps.shape[1] else None
        out[f"mask{s}"] = (is_repair[selected].astype(np.uint8)
                           if not compact and maps.shape[1] else None)
        out[f"prefix{s}"] = int(np.count_nonzero(in_prefix & selected))
    return out
