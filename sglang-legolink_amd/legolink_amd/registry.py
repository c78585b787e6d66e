"""Registered KV blocks: the supplier of the link's source slots.

A small registry with the LegoLink block registry's interface names
(patched_sglang_files/python/sglang/srt/mem_cache/radix_cache.py:
``register_legolink_block`` :755, ``get_legolink_block_tokens`` :950,
``lookup_legolink_blocks`` :995, ``acquire_legolink_blocks`` :1246,
``release_legolink_blocks`` :1330) and the handle fields the link reads
(``LegoLinkBlockHandle`` :289-334: token ids, ``kv_slots``,
``compile_local_positions``, pin count).  The radix tree, eviction policy,
compatibility keys and statistics of the reference registry manage block
lifetime, not link arithmetic, and are not restated.
"""

from __future__ import annotations

import operator
import threading
from dataclasses import dataclass, field
from typing import Any, Iterable, Optional, Sequence

import numpy as np
import torch


@dataclass
class LegoLinkBlockHandle:
    cache_key: str
    token_ids: tuple[int, ...]
    kv_slots: torch.Tensor                 # int64 [token_count], slots holding the block's K/V
    compile_local_positions: tuple[int, ...]  # RoPE positions the cached K carries
    block_id: str = ""
    # "reference": kv_slots index the KV pool; "clone": they index the snapshot
    # arena the block was copied into (pic_runtime.py:1985-1991, :3519-3527).
    storage_mode: str = "reference"
    pin_count: int = 0
    generation: int = 0
    valid: bool = True
    stale_reason: Optional[str] = None
    # Derived at registration: local position of token 0 when the positions
    # are consecutive (None otherwise), and their maximum (-1 when empty).
    local_start: Optional[int] = 0
    max_local_position: int = -1
    # Per-device copies the link reads (int64 slots; non-consecutive positions).
    _device_tensors: dict = field(default_factory=dict, repr=False, compare=False)
    # Row of the handle in its registry's per-device record tables.
    row: int = -1

    @property
    def token_count(self) -> int:
        return len(self.token_ids)

    def link_record(self, device: torch.device) -> tuple[int, int, int, int, int, int]:
        """(token count, address of the int64 slots on ``device``, address of the
        int64 compile-time positions or 0 when consecutive, local position of
        token 0, source set (1: snapshot arena), largest local position) --
        what a link reads per block, cached per device."""

        key = ("record", device.type, device.index)
        record = self._device_tensors.get(key)
        if record is None:
            local = self.local_positions_on(device)
            record = (self.token_count, self.slots_on(device).data_ptr(),
                      0 if local is None else local.data_ptr(),
                      0 if self.local_start is None else self.local_start,
                      1 if self.storage_mode == "clone" else 0, self.max_local_position)
            self._device_tensors[key] = record
        return record

    def slots_on(self, device: torch.device) -> torch.Tensor:
        """``kv_slots`` as a contiguous int64 tensor on ``device`` (cached)."""

        key = ("slots", str(device))
        cached = self._device_tensors.get(key)
        if cached is None:
            cached = self.kv_slots.to(device=device, dtype=torch.int64).contiguous()
            self._device_tensors[key] = cached
        return cached

    def local_positions_on(self, device: torch.device) -> Optional[torch.Tensor]:
        """The compile-time positions as an int64 tensor on ``device``, or None
        when they are consecutive (``local_start + i``)."""

        if self.local_start is not None:
            return None
        key = ("local", str(device))
        cached = self._device_tensors.get(key)
        if cached is None:
            cached = torch.tensor(self.compile_local_positions, dtype=torch.int64, device=device)
            self._device_tensors[key] = cached
        return cached


@dataclass
class LegoLinkLookupResult:
    matched_blocks: dict[str, LegoLinkBlockHandle] = field(default_factory=dict)
    kv_slot_ranges: dict[str, torch.Tensor] = field(default_factory=dict)
    missing_blocks: list[str] = field(default_factory=list)
    stale_blocks: list[str] = field(default_factory=list)
    matched_handles: list[LegoLinkBlockHandle] = field(default_factory=list)


def _int_array(values: Any) -> np.ndarray:
    """A flat int64 array of ``values`` (a range, list, array or tensor)."""

    if isinstance(values, range):
        return np.arange(values.start, values.stop, values.step, dtype=np.int64)
    if isinstance(values, torch.Tensor):
        return values.detach().reshape(-1).to("cpu", torch.int64).numpy()
    array = np.asarray(values)
    if array.size and not np.issubdtype(array.dtype, np.integer):
        array = np.asarray([int(value) for value in values], dtype=np.int64)
    return array.astype(np.int64, copy=False).reshape(-1)


_ROW = operator.attrgetter("row")


def _int_tuple(values: Any) -> tuple[int, ...]:
    return tuple(_int_array(values).tolist())


class LegoLinkBlockRegistry:
    """cache_key -> handle.  Callers on several threads are serialised by a lock."""

    def __init__(self) -> None:
        self._blocks: dict[str, LegoLinkBlockHandle] = {}
        self._lock = threading.Lock()
        self._generation = 0
        # Rows of the per-device record tables: a new handle takes an evicted
        # handle's row before a new one, so the tables stay as large as the
        # most handles ever registered at once.
        self._rows = 0
        self._free_rows: list[int] = []
        # Per device: the link records of every handle by row, and which rows are filled.
        self._records: dict[tuple[str, Optional[int]], tuple[np.ndarray, np.ndarray]] = {}

    def register_legolink_block(
        self,
        cache_key: str,
        token_ids: Sequence[int],
        kv_slots: torch.Tensor,
        *,
        compile_local_positions: Optional[Sequence[int]] = None,
        block_id: Optional[str] = None,
        storage_mode: str = "reference",
    ) -> LegoLinkBlockHandle:
        token_ids = _int_tuple(token_ids)
        slots = torch.as_tensor(kv_slots).long().reshape(-1).clone()
        if int(slots.numel()) != len(token_ids):
            raise ValueError("LegoLink KV slot count must equal the exact logical token length.")
        if compile_local_positions is None:
            position_array = np.arange(len(token_ids), dtype=np.int64)
        else:
            position_array = _int_array(compile_local_positions)
        positions = tuple(position_array.tolist())
        if len(positions) != len(token_ids):
            raise ValueError("compile_local_positions must hold one position per token.")
        if storage_mode not in ("reference", "clone"):
            raise ValueError(f"Unsupported PIC storage mode: {storage_mode}")
        if position_array.size == 0:
            local_start, max_local = 0, -1
        else:
            consecutive = bool(np.array_equal(
                position_array, position_array[0] + np.arange(position_array.size, dtype=np.int64)))
            local_start = int(position_array[0]) if consecutive else None
            max_local = int(position_array.max())
        with self._lock:
            resident = self._blocks.get(str(cache_key))
            if resident is not None and resident.valid:
                raise ValueError(f"LegoLink block {cache_key} is already registered.")
            self._generation += 1
            handle = LegoLinkBlockHandle(
                cache_key=str(cache_key),
                token_ids=token_ids,
                kv_slots=slots,
                compile_local_positions=positions,
                block_id=str(block_id or cache_key),
                generation=self._generation,
                storage_mode=storage_mode,
                local_start=local_start,
                max_local_position=max_local,
                row=self._take_row(),
            )
            self._blocks[str(cache_key)] = handle
            return handle

    def _take_row(self) -> int:
        if self._free_rows:
            return self._free_rows.pop()
        self._rows += 1
        return self._rows - 1

    @property
    def record_rows(self) -> int:
        """Rows the per-device record tables hold (live handles at most, at their peak)."""

        return self._rows

    def get_legolink_block_tokens(self, cache_key: str) -> Optional[tuple[int, ...]]:
        handle = self._blocks.get(str(cache_key))
        return handle.token_ids if handle is not None and handle.valid else None

    def lookup_legolink_blocks(self, cache_keys: Iterable[str]) -> LegoLinkLookupResult:
        result = LegoLinkLookupResult()
        with self._lock:
            for cache_key in (str(key) for key in cache_keys):
                handle = self._blocks.get(cache_key)
                if handle is None:
                    result.missing_blocks.append(cache_key)
                elif not handle.valid:
                    result.stale_blocks.append(cache_key)
                else:
                    result.matched_blocks[cache_key] = handle
                    result.kv_slot_ranges[cache_key] = handle.kv_slots
                    result.matched_handles.append(handle)
        return result

    def link_handles(self, cache_keys: Sequence[str]) -> tuple[list[Optional[LegoLinkBlockHandle]], list[str]]:
        """The valid handle of every key, in order (None where missing or
        stale), and the keys that cannot be linked: ``lookup_legolink_blocks``
        reduced to what a link reads, in one pass."""

        with self._lock:
            handles = list(map(self._blocks.get, cache_keys))
        unavailable = [str(key) for key, handle in zip(cache_keys, handles) if handle is None or not handle.valid]
        return handles, unavailable

    def link_records(self, handles: Sequence[LegoLinkBlockHandle], device: torch.device) -> np.ndarray:
        """int64 ``[len(handles), 6]``: every handle's ``link_record(device)``,
        gathered from a per-device table (filled once per handle and device),
        so that a link of many blocks reads them with one index."""

        key = (device.type, device.index)
        with self._lock:
            rows = np.fromiter(map(_ROW, handles), dtype=np.int64, count=len(handles))
            if rows.size and int(rows.min()) < 0:
                stale = next(handle for handle in handles if handle.row < 0)
                raise ValueError(f"LegoLink block {stale.cache_key} was evicted; it has no link record.")
            table, filled = self._records.get(key, (None, None))
            if table is None or table.shape[0] < self._rows:
                capacity = max(64, 2 * self._rows)
                grown = np.zeros((capacity, 6), dtype=np.int64)
                grown_filled = np.zeros(capacity, dtype=bool)
                if table is not None:
                    grown[: table.shape[0]] = table
                    grown_filled[: filled.shape[0]] = filled
                table, filled = grown, grown_filled
                self._records[key] = (table, filled)
            missing = np.flatnonzero(~filled[rows])
            for index in missing.tolist():
                handle = handles[index]
                table[handle.row] = handle.link_record(device)
                filled[handle.row] = True
            return table[rows]

    def acquire_legolink_blocks(self, handles: Iterable[LegoLinkBlockHandle]) -> list[LegoLinkBlockHandle]:
        handles = list(handles)
        with self._lock:
            for handle in handles:
                handle.pin_count += 1
        return handles

    def release_legolink_blocks(self, handles: Iterable[LegoLinkBlockHandle]) -> None:
        with self._lock:
            for handle in handles:
                if handle.pin_count <= 0:
                    raise ValueError(f"LegoLink block {handle.cache_key} is not pinned.")
                handle.pin_count -= 1

    def evict_legolink_block(self, cache_key: str) -> Optional[LegoLinkBlockHandle]:
        """Invalidate an unpinned block and return its handle (so the caller can
        free its slots); pinned blocks stay resident and None is returned."""

        with self._lock:
            handle = self._blocks.get(str(cache_key))
            if handle is None or handle.pin_count > 0 or not handle.valid:
                return None
            handle.valid = False
            handle.stale_reason = "evicted"
            # The handle stays (lookups report it stale); its record row and
            # its per-device copies of the slots and positions are released.
            if handle.row >= 0:
                for _, filled in self._records.values():
                    if handle.row < filled.shape[0]:
                        filled[handle.row] = False
                self._free_rows.append(handle.row)
                handle.row = -1
            handle._device_tensors.clear()
            return handle
