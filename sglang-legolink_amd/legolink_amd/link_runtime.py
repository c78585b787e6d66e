"""The batched link executor: registered blocks -> a new request's KV slots.

Host side of the reference's ``PICRuntime._copy_linked_kv`` and
``_copy_linked_kv_batched_blocks``
(patched_sglang_files/python/sglang/srt/pic_runtime.py:4593-4729 and
:4881-5013, 5153-5208): validate the pool, look up the blocks of the plan,
build the concatenated source/destination/local/global maps in plan order,
find the identity prefix and the repair rows, then run the HIP link over every
layer.  Where the reference calls its fused operator once per layer, one
prepared launch covers all layers.

Differences that keep the result identical:
* repair rows (``imp_indices`` inside blocks) are dropped from the maps instead
  of being passed as a mask when ``compact_repair_rows`` is on (no empty waves);
* a block's compile-time positions come from its registry handle
  (``compile_local_positions``, radix_cache.py:892) instead of being assumed to
  be 0..n-1, so blocks compiled behind a prefix remap correctly.
"""

from __future__ import annotations

import os
import time
from dataclasses import dataclass, field
from typing import Any, Mapping, Optional, Sequence

import numpy as np
import torch

from . import kv_link
from .errors import LinkRuntimeError
from .registry import LegoLinkBlockRegistry
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
    the link kernel on the current stream, ``write_repaired()`` the repaired-row
    write-back of the rows the link skipped."""

    def __init__(self, *, pool: Any, layers: list[int], maps: LinkMaps, groups: list[tuple[list[int], RotarySpec]],
                 boundary_repair_aware: bool, compact_repair_rows: bool, num_warps: Optional[int],
                 layers_per_wave: int, validate_indices: bool) -> None:
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
        mask_tensor = None
        prefix = maps.prefix_token_count
        if repair.size and compact_repair_rows:
            keep = np.ones(token_count, dtype=bool)
            keep[repair] = False
            keep_index = np.flatnonzero(keep)
            keep_device = torch.from_numpy(keep_index).to(device)
            source = maps.source_slots.index_select(0, keep_device)
            destination = maps.destination_slots.index_select(0, keep_device)
            local = maps.local_positions[keep_index]
            global_ = maps.global_positions[keep_index]
            prefix = int(np.count_nonzero(keep[:prefix]))
        else:
            source, destination = maps.source_slots, maps.destination_slots
            local, global_ = maps.local_positions, maps.global_positions
            if repair.size:
                mask = np.zeros(token_count, dtype=np.uint8)
                mask[repair] = 1
                mask_tensor = torch.from_numpy(mask).to(device)
        positions = torch.from_numpy(np.stack((local, global_))).to(device)
        self.source_slots, self.destination_slots = source, destination
        self.local_positions, self.global_positions = positions[0], positions[1]
        self.repair_mask = mask_tensor
        self.prefix_token_count = prefix
        self.linked_token_count = int(source.numel())
        self._links: list[kv_link.PreparedKVLink] = []
        if self.linked_token_count:
            index_of = {layer: i for i, layer in enumerate(layers)}
            for group_layers, rotary in groups:
                self._links.append(kv_link.PreparedKVLink(
                    key_buffers=[key_buffers[index_of[layer]] for layer in group_layers],
                    value_buffers=[value_buffers[index_of[layer]] for layer in group_layers],
                    source_slots=source,
                    destination_slots=destination,
                    local_positions=self.local_positions,
                    global_positions=self.global_positions,
                    cos_sin_cache=rotary.cos_sin_cache,
                    prefix_token_count=prefix,
                    rotary_dim=rotary.rotary_dim,
                    is_neox_style=rotary.is_neox_style,
                    repair_mask=mask_tensor,
                    num_warps=num_warps,
                    layers_per_wave=layers_per_wave,
                    validate_indices=validate_indices,
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
            **self.traffic,
        }


class KVLinkExecutor:
    """Links registered blocks into request slots on one GPU."""

    def __init__(self, registry: LegoLinkBlockRegistry, rotary: RotarySpec | Mapping[int, RotarySpec], *,
                 start_layer: int = 0, end_layer: int, num_warps: Optional[int] = None,
                 layers_per_wave: int = 0) -> None:
        self.registry = registry
        self.start_layer = int(start_layer)
        self.end_layer = int(end_layer)
        if isinstance(rotary, RotarySpec):
            self.rotary_by_layer = {layer: rotary for layer in range(self.start_layer, self.end_layer)}
        else:
            self.rotary_by_layer = dict(rotary)
        self.num_warps = num_warps
        self.layers_per_wave = layers_per_wave

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
        sources, destinations, locals_, globals_, repair_offsets, specs = [], [], [], [], [], []
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
            inside = repair_array[(repair_array >= start) & (repair_array < end)]
            repair_offsets.append(offset + inside - start)
            specs.append({
                "block_index": block_index,
                "cache_key": cache_key,
                "start": start,
                "end": end,
                "token_count": count,
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
        )

    # -- link ---------------------------------------------------------------
    def _layer_groups(self, layers: list[int], max_position: int) -> list[tuple[list[int], RotarySpec]]:
        groups: list[tuple[list[int], RotarySpec]] = []
        for layer in layers:
            rotary = self.rotary_by_layer.get(layer)
            if rotary is None:
                raise LinkRuntimeError(f"Layer {layer} has no supported rotary embedding for PIC.")
            rotary.ensure_cos_sin_cache_length(max_position)
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
        maps = self.build_link_maps(destination_slots, link_plan,
                                    device=pool.get_key_buffer(self.start_layer).device)
        layers = list(range(self.start_layer, self.end_layer))
        max_position = int(max(maps.local_positions.max(), maps.global_positions.max()))
        # Positions of prefix tokens are never read, but a table that covers
        # every position keeps validation simple.
        groups = self._layer_groups(layers, max_position)
        for rotary in self.rotary_by_layer.values():
            if rotary.cos_sin_cache.device != maps.destination_slots.device:
                rotary.cos_sin_cache = rotary.cos_sin_cache.to(maps.destination_slots.device)
        prepared = PreparedLink(
            pool=pool, layers=layers, maps=maps, groups=groups,
            boundary_repair_aware=bool(boundary_repair_aware), compact_repair_rows=compact_repair_rows,
            num_warps=self.num_warps, layers_per_wave=self.layers_per_wave,
            validate_indices=validate_indices,
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
        layers = range(self.start_layer, self.end_layer)
        kv_link.scatter_kv_rows_inplace(
            key_buffers=[pool.get_key_buffer(layer) for layer in layers],
            value_buffers=[pool.get_value_buffer(layer) for layer in layers],
            destination_slots=destination_slots.index_select(0, index),
            repaired_keys=repaired_keys,
            repaired_values=repaired_values,
        )
