"""The batched link executor: registered blocks -> a new request's KV slots.

Host side of the reference's ``PICRuntime._copy_linked_kv`` and
``_copy_linked_kv_batched_blocks``
(patched_sglang_files/python/sglang/srt/pic_runtime.py:4593-4729 and
:4881-5013, 5153-5208): validate the pool, look up the blocks of the plan,
build the concatenated source/destination/local/global maps in plan order,
find the identity prefix and the repair rows, then run the HIP link over every
layer.  Where the reference calls its fused operator once per layer, one
prepared launch covers all layers.

Also here, all on the same kernel:
* block capture (``capture_compile_blocks``, pic_runtime.py:3485-3560):
  "reference" blocks keep their pool slots, "clone" blocks are copied into a
  snapshot arena -- one per-layer buffer with the pool's row layout instead of
  a tensor per block and layer;
* links that mix reference and clone blocks (pic_runtime.py:5553-5567): one
  launch per source (pool or arena);
* group promotion (``_promote_reconstructed_group``, pic_runtime.py:5901-5922):
  a linked range copied into new slots with K rotated from its global
  positions back to 0..n-1.

Differences from the reference that keep the result identical:
* repair rows (``imp_indices`` inside blocks) are dropped from the maps instead
  of being passed as a mask when ``compact_repair_rows`` is on (no empty waves);
* a block's compile-time positions come from its registry handle
  (``compile_local_positions``, radix_cache.py:892) instead of being assumed to
  be 0..n-1, so blocks compiled behind a prefix remap correctly.
"""

from __future__ import annotations

import os
import threading
import time
from dataclasses import dataclass, field
from typing import Any, Mapping, Optional, Sequence

import numpy as np
import torch

from . import kv_link
from .errors import LinkRuntimeError
from .registry import LegoLinkBlockHandle, LegoLinkBlockRegistry
from .rope import RotarySpec


def _env_flag(name: str, default: str) -> bool:
    return os.getenv(name, default).strip().lower() in ("1", "true", "yes", "on")


class KVPool:
    """MHA KV pool: one dense [slots, heads, dim] K and V buffer per layer
    (the layout of SGLang's MHA token-to-KV pool; layers are separate
    allocations)."""

    def __init__(self, key_buffers: Sequence[torch.Tensor], value_buffers: Sequence[torch.Tensor],
                 *, start_layer: int = 0) -> None:
        if not key_buffers or len(key_buffers) != len(value_buffers):
            raise ValueError("a pool needs one K and one V buffer per layer")
        self.k_buffer = list(key_buffers)
        self.v_buffer = list(value_buffers)
        self.start_layer = int(start_layer)
        self.dtype = self.k_buffer[0].dtype
        self.store_dtype = self.dtype
        self.size = int(self.k_buffer[0].shape[0])
        self.layer_num = len(self.k_buffer)

    @classmethod
    def allocate(cls, *, num_slots: int, num_layers: int, num_heads: int, head_dim: int,
                 value_head_dim: Optional[int] = None, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cuda", start_layer: int = 0) -> "KVPool":
        value_head_dim = head_dim if value_head_dim is None else value_head_dim
        keys = [torch.empty(num_slots, num_heads, head_dim, dtype=dtype, device=device)
                for _ in range(num_layers)]
        values = [torch.empty(num_slots, num_heads, value_head_dim, dtype=dtype, device=device)
                  for _ in range(num_layers)]
        return cls(keys, values, start_layer=start_layer)

    def get_key_buffer(self, layer_id: int) -> torch.Tensor:
        return self.k_buffer[layer_id - self.start_layer]

    def get_value_buffer(self, layer_id: int) -> torch.Tensor:
        return self.v_buffer[layer_id - self.start_layer]


class SnapshotArena(KVPool):
    """Storage of clone-mode blocks: the pool's row layout, with a first-fit
    allocator of contiguous slot ranges (one range per block)."""

    def __init__(self, key_buffers: Sequence[torch.Tensor], value_buffers: Sequence[torch.Tensor],
                 *, start_layer: int = 0) -> None:
        super().__init__(key_buffers, value_buffers, start_layer=start_layer)
        self._free: list[tuple[int, int]] = [(0, self.size)]  # sorted (start, length)
        self._lock = threading.Lock()

    @property
    def free_slots(self) -> int:
        return sum(length for _, length in self._free)

    def alloc(self, count: int) -> Optional[torch.Tensor]:
        """``count`` consecutive slots, or None when no free range is long enough."""

        count = int(count)
        if count <= 0:
            raise ValueError("count must be positive")
        with self._lock:
            for index, (start, length) in enumerate(self._free):
                if length >= count:
                    if length == count:
                        self._free.pop(index)
                    else:
                        self._free[index] = (start + count, length - count)
                    return torch.arange(start, start + count, dtype=torch.long,
                                        device=self.k_buffer[0].device)
        return None

    def free(self, slots: torch.Tensor) -> None:
        """Return a range obtained from ``alloc``."""

        values = slots.detach().cpu().numpy()
        if values.size == 0:
            return
        start, count = int(values[0]), int(values.size)
        if not np.array_equal(values, np.arange(start, start + count)):
            raise ValueError("arena slots are freed as the range alloc returned")
        with self._lock:
            for free_start, length in self._free:
                if start < free_start + length and free_start < start + count:
                    raise ValueError("arena range is already free")
            self._free.append((start, count))
            self._free.sort()
            merged: list[tuple[int, int]] = []
            for free_start, length in self._free:
                if merged and merged[-1][0] + merged[-1][1] == free_start:
                    merged[-1] = (merged[-1][0], merged[-1][1] + length)
                else:
                    merged.append((free_start, length))
            self._free = merged


@dataclass
class LinkMaps:
    """Token maps of one link in plan order (before compaction)."""

    source_slots: torch.Tensor        # int64 [T] on the pool device
    destination_slots: torch.Tensor   # int64 [T] on the pool device
    local_positions: np.ndarray       # int64 [T]
    global_positions: np.ndarray      # int64 [T]
    repair_offsets: np.ndarray        # int64 [R] token offsets of repair rows (sorted)
    prefix_token_count: int
    block_specs: list[dict[str, Any]] = field(default_factory=list)
    clone_tokens: Optional[np.ndarray] = None  # bool [T]: token's block is clone-mode

    @property
    def token_count(self) -> int:
        return int(self.local_positions.shape[0])


def _validate_pool(pool: Any) -> None:
    """pic_runtime.py:6283-6289."""

    if not all(hasattr(pool, method) for method in ("get_key_buffer", "get_value_buffer")):
        raise LinkRuntimeError("PIC link requires an MHA-style KV pool.")
    if getattr(pool, "store_dtype", None) != getattr(pool, "dtype", None):
        raise LinkRuntimeError("PIC link does not yet support quantized KV cache.")


class PreparedLink:
    """One link, validated and with its device maps built; ``launch()`` enqueues
    the link kernel(s) on the current stream, ``write_repaired()`` the
    repaired-row write-back of the rows the link skipped."""

    def __init__(self, *, pool: Any, layers: list[int], maps: LinkMaps,
                 groups: list[tuple[list[int], RotarySpec]], boundary_repair_aware: bool,
                 compact_repair_rows: bool, num_warps: Optional[int], layers_per_wave: int,
                 validate_indices: bool, arena: Optional[SnapshotArena] = None) -> None:
        self.pool = pool
        self.layers = layers
        self.maps = maps
        self.host_prepare_s = 0.0
        self.boundary_repair_aware = boundary_repair_aware
        device = maps.destination_slots.device
        key_buffers = [pool.get_key_buffer(layer) for layer in layers]
        value_buffers = [pool.get_value_buffer(layer) for layer in layers]
        self.key_buffers, self.value_buffers = key_buffers, value_buffers
        token_count = maps.token_count
        repair = maps.repair_offsets if boundary_repair_aware else np.zeros(0, dtype=np.int64)
        self.repair_offsets = repair
        self.repair_destination_slots = maps.destination_slots.index_select(
            0, torch.from_numpy(repair).to(device)
        ) if repair.size else maps.destination_slots[:0]
        clone = maps.clone_tokens if maps.clone_tokens is not None else np.zeros(token_count, dtype=bool)
        if clone.any() and arena is None:
            raise LinkRuntimeError("PIC link of clone-mode blocks needs the snapshot arena.")
        is_repair = np.zeros(token_count, dtype=bool)
        is_repair[repair] = True
        # One launch per source: the pool (reference blocks), the arena (clone blocks).
        sources: list[tuple[np.ndarray, Optional[SnapshotArena]]] = []
        for from_arena in (False, True):
            members = clone if from_arena else ~clone
            if members.any():
                sources.append((members, arena if from_arena else None))
        self._links: list[kv_link.PreparedKVLink] = []
        self._keepalive: list[Any] = []
        self.linked_token_count = 0
        index_of = {layer: i for i, layer in enumerate(layers)}
        for members, source_arena in sources:
            if compact_repair_rows:
                selected = np.flatnonzero(members & ~is_repair)
                mask_tensor = None
            else:
                selected = np.flatnonzero(members)
                mask_tensor = (torch.from_numpy(is_repair[selected].astype(np.uint8)).to(device)
                               if is_repair[selected].any() else None)
            if selected.size == 0:
                continue
            prefix = int(np.count_nonzero(selected < maps.prefix_token_count))
            selected_device = torch.from_numpy(selected).to(device)
            source = maps.source_slots.index_select(0, selected_device)
            destination = maps.destination_slots.index_select(0, selected_device)
            positions = torch.from_numpy(np.stack((maps.local_positions[selected],
                                                   maps.global_positions[selected]))).to(device)
            self._keepalive.append((source, destination, positions, mask_tensor))
            self.linked_token_count += int(np.count_nonzero(~is_repair[selected]))
            for group_layers, rotary in groups:
                indices = [index_of[layer] for layer in group_layers]
                self._links.append(kv_link.PreparedKVLink(
                    key_buffers=[key_buffers[i] for i in indices],
                    value_buffers=[value_buffers[i] for i in indices],
                    source_slots=source,
                    destination_slots=destination,
                    local_positions=positions[0],
                    global_positions=positions[1],
                    cos_sin_cache=rotary.cos_sin_cache,
                    prefix_token_count=prefix,
                    rotary_dim=rotary.rotary_dim,
                    is_neox_style=rotary.is_neox_style,
                    repair_mask=mask_tensor,
                    num_warps=num_warps,
                    layers_per_wave=layers_per_wave,
                    validate_indices=validate_indices,
                    source_key_buffers=(None if source_arena is None else
                                        [source_arena.get_key_buffer(layer) for layer in group_layers]),
                    source_value_buffers=(None if source_arena is None else
                                          [source_arena.get_value_buffer(layer) for layer in group_layers]),
                ))
        key_row = int(key_buffers[0][0].numel()) * key_buffers[0].element_size()
        value_row = int(value_buffers[0][0].numel()) * value_buffers[0].element_size()
        self.traffic = kv_link.estimate_kv_traffic_bytes(
            token_count=token_count,
            key_row_bytes=key_row,
            value_row_bytes=value_row,
            remapped_token_count=token_count - maps.prefix_token_count,
            repair_token_count=int(repair.size),
        )
        self.algorithmic_link_bytes = self.linked_token_count * (key_row + value_row) * 2 * len(layers)

    @property
    def launch_info(self) -> list[dict[str, int]]:
        return [link.launch for link in self._links]

    def launch(self, stream: torch.cuda.Stream | None = None) -> None:
        for link in self._links:
            link(stream)

    def write_repaired(self, repaired_keys: torch.Tensor, repaired_values: torch.Tensor,
                       stream: torch.cuda.Stream | None = None) -> None:
        """K_l[dst of repair row r] = repaired_keys[l, r] for the repair rows inside
        blocks, in request-position order ([layers, rows, heads, dim])."""

        self.prepare_write_repaired(repaired_keys, repaired_values)(stream)

    def prepare_write_repaired(self, repaired_keys: torch.Tensor,
                               repaired_values: torch.Tensor) -> kv_link.PreparedKVScatter:
        return kv_link.PreparedKVScatter(
            key_buffers=self.key_buffers,
            value_buffers=self.value_buffers,
            destination_slots=self.repair_destination_slots,
            repaired_keys=repaired_keys,
            repaired_values=repaired_values,
        )

    def record(self) -> dict[str, Any]:
        return {
            "token_count": self.maps.token_count,
            "linked_token_count": self.linked_token_count,
            "block_count": len(self.maps.block_specs),
            "prefix_token_count": self.maps.prefix_token_count,
            "remapped_token_count": self.maps.token_count - self.maps.prefix_token_count,
            "repair_token_count": int(self.repair_offsets.size),
            "boundary_repair_aware": self.boundary_repair_aware,
            "layers_written": len(self.layers),
            "kernel_launches": sum(info["launches"] for info in self.launch_info),
            "launch": self.launch_info,
            "rope_remapped": [spec["needs_rope_remap"] for spec in self.maps.block_specs],
            "storage_modes": [spec["storage_mode"] for spec in self.maps.block_specs],
            **self.traffic,
        }


class KVLinkExecutor:
    """Links registered blocks into request slots on one GPU."""

    def __init__(self, registry: LegoLinkBlockRegistry, rotary: RotarySpec | Mapping[int, RotarySpec], *,
                 start_layer: int = 0, end_layer: int, num_warps: Optional[int] = None,
                 layers_per_wave: int = 0, arena: Optional[SnapshotArena] = None) -> None:
        self.registry = registry
        self.start_layer = int(start_layer)
        self.end_layer = int(end_layer)
        if isinstance(rotary, RotarySpec):
            self.rotary_by_layer = {layer: rotary for layer in range(self.start_layer, self.end_layer)}
        else:
            self.rotary_by_layer = dict(rotary)
        self.num_warps = num_warps
        self.layers_per_wave = layers_per_wave
        self.arena = arena

    @property
    def layers(self) -> list[int]:
        return list(range(self.start_layer, self.end_layer))

    # -- maps ---------------------------------------------------------------
    def build_link_maps(self, destination_slots: torch.Tensor, link_plan: Mapping[str, Any],
                        *, device: Optional[torch.device] = None) -> LinkMaps:
        """Concatenated maps in plan order (pic_runtime.py:4911-5013)."""

        ranges = link_plan.get("block_ranges") or link_plan.get("attention_ranges")
        cache_keys = link_plan.get("cache_keys")
        if not isinstance(ranges, list) or not isinstance(cache_keys, list):
            raise LinkRuntimeError("PIC link plan is missing block ranges/cache keys.")
        if len(ranges) != len(cache_keys):
            raise LinkRuntimeError("PIC block range and cache key counts differ.")
        if not cache_keys:
            raise LinkRuntimeError("PIC link plan has no blocks.")
        lookup = self.registry.lookup_legolink_blocks(str(key) for key in cache_keys)
        unavailable = [*lookup.missing_blocks, *lookup.stale_blocks]
        if unavailable:
            raise LinkRuntimeError(
                f"PIC RadixCache lookup cannot safely link block(s): {', '.join(unavailable)}"
            )
        device = destination_slots.device if device is None else device
        repair_positions = sorted({int(p) for p in (link_plan.get("imp_indices") or [])})
        repair_array = np.asarray(repair_positions, dtype=np.int64)
        sources, destinations, locals_, globals_, repair_offsets, clones, specs = [], [], [], [], [], [], []
        offset = 0
        for block_index, (block_range, raw_key) in enumerate(zip(ranges, cache_keys)):
            cache_key = str(raw_key)
            handle = lookup.matched_blocks[cache_key]
            start, end = int(block_range["start_token"]), int(block_range["end_token"])
            count = end - start
            if count != handle.token_count:
                raise LinkRuntimeError(
                    f"PIC token count mismatch for block {cache_key}: plan={count}, "
                    f"snapshot={handle.token_count}"
                )
            if end > int(destination_slots.numel()) or start < 0:
                raise LinkRuntimeError(f"PIC block {cache_key} range exceeds the request's slots.")
            local = np.asarray(handle.compile_local_positions, dtype=np.int64)
            global_ = np.arange(start, end, dtype=np.int64)
            sources.append(handle.kv_slots.to(device, non_blocking=True))
            destinations.append(destination_slots[start:end])
            locals_.append(local)
            globals_.append(global_)
            clones.append(np.full(count, handle.storage_mode == "clone"))
            inside = repair_array[(repair_array >= start) & (repair_array < end)]
            repair_offsets.append(offset + inside - start)
            specs.append({
                "block_index": block_index,
                "cache_key": cache_key,
                "start": start,
                "end": end,
                "token_count": count,
                "storage_mode": handle.storage_mode,
                "needs_rope_remap": bool(np.any(local != global_)),
                "repair_token_count": int(inside.size),
            })
            offset += count
        first = specs[0]
        prefix = 0 if first["needs_rope_remap"] else int(first["token_count"])
        return LinkMaps(
            source_slots=torch.cat(sources).long(),
            destination_slots=torch.cat(destinations).to(device).long(),
            local_positions=np.concatenate(locals_),
            global_positions=np.concatenate(globals_),
            repair_offsets=np.concatenate(repair_offsets).astype(np.int64),
            prefix_token_count=prefix,
            block_specs=specs,
            clone_tokens=np.concatenate(clones),
        )

    # -- link ---------------------------------------------------------------
    def _layer_groups(self, layers: list[int], max_position: int,
                      device: torch.device) -> list[tuple[list[int], RotarySpec]]:
        groups: list[tuple[list[int], RotarySpec]] = []
        for layer in layers:
            rotary = self.rotary_by_layer.get(layer)
            if rotary is None:
                raise LinkRuntimeError(f"Layer {layer} has no supported rotary embedding for PIC.")
            rotary.ensure_cos_sin_cache_length(max_position)
            if rotary.cos_sin_cache.device != device:
                rotary.cos_sin_cache = rotary.cos_sin_cache.to(device)
            for group_layers, group_rotary in groups:
                if group_rotary is rotary:
                    group_layers.append(layer)
                    break
            else:
                groups.append(([layer], rotary))
        return groups

    def prepare_link(self, pool: Any, destination_slots: torch.Tensor, link_plan: Mapping[str, Any], *,
                     boundary_repair_aware: Optional[bool] = None, compact_repair_rows: bool = True,
                     validate_indices: bool = False) -> PreparedLink:
        started = time.perf_counter()
        _validate_pool(pool)
        if boundary_repair_aware is None:
            boundary_repair_aware = _env_flag("SGLANG_PIC_TRITON_BOUNDARY_REPAIR_AWARE", "0")
        device = pool.get_key_buffer(self.start_layer).device
        maps = self.build_link_maps(destination_slots, link_plan, device=device)
        max_position = int(max(maps.local_positions.max(), maps.global_positions.max()))
        groups = self._layer_groups(self.layers, max_position, device)
        prepared = PreparedLink(
            pool=pool, layers=self.layers, maps=maps, groups=groups,
            boundary_repair_aware=bool(boundary_repair_aware), compact_repair_rows=compact_repair_rows,
            num_warps=self.num_warps, layers_per_wave=self.layers_per_wave,
            validate_indices=validate_indices, arena=self.arena,
        )
        prepared.host_prepare_s = time.perf_counter() - started
        return prepared

    def copy_linked_kv(self, pool: Any, destination_slots: torch.Tensor, link_plan: Mapping[str, Any],
                       **options: Any) -> dict[str, Any]:
        """Link the plan's blocks into ``destination_slots`` (the request's slots
        indexed by request position) on the current stream; returns an
        accounting record.  Blocks stay pinned while the link is enqueued."""

        lookup = self.registry.lookup_legolink_blocks(str(key) for key in link_plan.get("cache_keys") or [])
        handles = self.registry.acquire_legolink_blocks(lookup.matched_handles)
        try:
            prepared = self.prepare_link(pool, destination_slots, link_plan, **options)
            prepared.launch()
        finally:
            self.registry.release_legolink_blocks(handles)
        record = prepared.record()
        record["host_prepare_s"] = prepared.host_prepare_s
        return record

    def write_repaired_kv(self, pool: Any, destination_slots: torch.Tensor, positions: Sequence[int],
                          repaired_keys: torch.Tensor, repaired_values: torch.Tensor) -> None:
        """Repair write-back: K_l[destination_slots[p]] = repaired_keys[l, i] for
        the i-th position p (flashinfer_sparse_repair.py:2235-2239)."""

        _validate_pool(pool)
        index = torch.as_tensor(list(positions), dtype=torch.long, device=destination_slots.device)
        kv_link.scatter_kv_rows_inplace(
            key_buffers=[pool.get_key_buffer(layer) for layer in self.layers],
            value_buffers=[pool.get_value_buffer(layer) for layer in self.layers],
            destination_slots=destination_slots.index_select(0, index),
            repaired_keys=repaired_keys,
            repaired_values=repaired_values,
        )

    # -- capture and promotion ------------------------------------------------
    def _any_rotary(self) -> RotarySpec:
        return self.rotary_by_layer[self.start_layer]

    def _copy_rows(self, *, destination: Any, source: Any, source_slots: torch.Tensor,
                   destination_slots: torch.Tensor, local: torch.Tensor, global_: torch.Tensor,
                   prefix: int) -> None:
        """One link launch between two pools (or within one) over every layer."""

        max_position = int(max(int(local.max()), int(global_.max()))) if prefix < local.numel() else 0
        groups = self._layer_groups(self.layers, max_position, source_slots.device)
        same_pool = source is destination
        for group_layers, rotary in groups:
            kv_link.fused_kv_link_layers_inplace(
                key_buffers=[destination.get_key_buffer(layer) for layer in group_layers],
                value_buffers=[destination.get_value_buffer(layer) for layer in group_layers],
                source_slots=source_slots,
                destination_slots=destination_slots,
                local_positions=local,
                global_positions=global_,
                cos_sin_cache=rotary.cos_sin_cache,
                prefix_token_count=prefix,
                rotary_dim=rotary.rotary_dim,
                is_neox_style=rotary.is_neox_style,
                num_warps=self.num_warps,
                layers_per_wave=self.layers_per_wave,
                source_key_buffers=None if same_pool else [source.get_key_buffer(layer) for layer in group_layers],
                source_value_buffers=None if same_pool else [source.get_value_buffer(layer) for layer in group_layers],
            )

    def capture_block(self, pool: Any, cache_key: str, token_ids: Sequence[int], slots: torch.Tensor, *,
                      storage_mode: str = "reference",
                      compile_local_positions: Optional[Sequence[int]] = None,
                      block_id: Optional[str] = None) -> LegoLinkBlockHandle:
        """Register a compiled block (capture_compile_blocks, pic_runtime.py:3485-3560).

        "reference": the block is read from ``slots`` of the pool when linked.
        "clone": its rows of every layer are copied bit for bit into the
        snapshot arena first, so the pool slots may be reused afterwards.
        """

        _validate_pool(pool)
        slots = torch.as_tensor(slots).long().reshape(-1).to(pool.get_key_buffer(self.start_layer).device)
        if storage_mode == "reference":
            return self.registry.register_legolink_block(
                cache_key, token_ids, slots, compile_local_positions=compile_local_positions,
                block_id=block_id, storage_mode="reference")
        if storage_mode != "clone":
            raise LinkRuntimeError(f"Unsupported PIC storage mode: {storage_mode}")
        if self.arena is None:
            raise LinkRuntimeError("PIC clone storage needs a snapshot arena.")
        count = int(slots.numel())
        arena_slots = self.arena.alloc(count)
        if arena_slots is None:
            raise LinkRuntimeError(f"PIC snapshot arena has no {count} free slots for {cache_key}.")
        try:
            positions = torch.zeros(count, dtype=torch.long, device=slots.device)
            self._copy_rows(destination=self.arena, source=pool, source_slots=slots,
                            destination_slots=arena_slots, local=positions, global_=positions,
                            prefix=count)
            return self.registry.register_legolink_block(
                cache_key, token_ids, arena_slots, compile_local_positions=compile_local_positions,
                block_id=block_id, storage_mode="clone")
        except Exception:
            self.arena.free(arena_slots)
            raise

    def release_block(self, cache_key: str) -> bool:
        """Evict an unpinned block; a clone block's arena range is freed."""

        handle = self.registry.evict_legolink_block(cache_key)
        if handle is None:
            return False
        if handle.storage_mode == "clone" and self.arena is not None:
            self.arena.free(handle.kv_slots)
        return True

    def promote_group(self, pool: Any, destination_slots: torch.Tensor, *, group_start: int,
                      group_end: int, new_slots: torch.Tensor, cache_key: str,
                      token_ids: Sequence[int]) -> LegoLinkBlockHandle:
        """Copy a linked request's rows [group_start, group_end) into ``new_slots``
        with K rotated from its global positions back to 0..n-1, and register
        the copy as a block (_promote_reconstructed_group,
        pic_runtime.py:5901-5922).  Like the reference, the rotation runs even
        when the group starts at position 0."""

        _validate_pool(pool)
        count = int(group_end) - int(group_start)
        if count <= 0 or group_start < 0 or group_end > int(destination_slots.numel()):
            raise LinkRuntimeError("PIC group promotion range exceeds the request's slots.")
        if len(token_ids) != count:
            raise LinkRuntimeError("PIC group promotion token count differs from its range.")
        new_slots = torch.as_tensor(new_slots).long().reshape(-1).to(destination_slots.device)
        if int(new_slots.numel()) != count:
            raise LinkRuntimeError("PIC group promotion needs one new slot per token.")
        device = destination_slots.device
        global_positions = torch.arange(group_start, group_end, dtype=torch.long, device=device)
        local_positions = torch.arange(count, dtype=torch.long, device=device)
        # global -> local: the inverse of what the next link of the block does.
        self._copy_rows(destination=pool, source=pool,
                        source_slots=destination_slots[group_start:group_end].contiguous(),
                        destination_slots=new_slots, local=global_positions, global_=local_positions,
                        prefix=0)
        return self.registry.register_legolink_block(cache_key, token_ids, new_slots,
                                                     storage_mode="reference")
