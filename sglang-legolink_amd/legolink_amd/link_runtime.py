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

Rounding of re-rotated K follows the reference's dispatch
(pic_runtime.py:1307-1323, :5033-5035, :5153-5165): with the fused mode off
(``SGLANG_PIC_TRITON_FUSED_KV_LINK`` = 0, its default) the reference runs its
torch path, so the link uses the "eager" rounding points; with the mode on
("1" / "auto") it uses the fused kernel's, unless a block is stored in clone
mode ("required" then fails, "auto" falls back to eager).  Group promotion is
always eager (``_remap_key_positions``, :5914-5919).  Both run on the same HIP
kernels.

Differences from the reference that keep the result identical:
* repair rows (``imp_indices`` inside blocks) are dropped from the maps instead
  of being passed as a mask when ``compact_repair_rows`` is on (no empty waves);
* a block's compile-time positions come from its registry handle
  (``compile_local_positions``, radix_cache.py:892) instead of being assumed to
  be 0..n-1, so blocks compiled behind a prefix remap correctly.
"""

from __future__ import annotations

import itertools
import operator
import os
import threading
import time
from dataclasses import dataclass
from typing import Any, Mapping, Optional, Sequence

import numpy as np
import torch

from . import _native, kv_link, link_maps
from .errors import LinkRuntimeError

try:
    from . import _host_sequences
except ImportError as error:  # the C module is built with the library
    raise ImportError("legolink_amd._host_sequences is not built: run `python -m legolink_amd.build` "
                      "from sglang-legolink_amd/") from error
from .registry import LegoLinkBlockHandle, LegoLinkBlockRegistry
from .rope import RotarySpec


def _env_flag(name: str, default: str) -> bool:
    return os.getenv(name, default).strip().lower() in ("1", "true", "yes", "on")


_FUSED_MODE_ALIASES = {
    "0": "disabled", "false": "disabled", "off": "disabled", "disabled": "disabled",
    "1": "required", "true": "required", "on": "required", "required": "required",
    "auto": "auto",
}


def get_fused_kv_link_mode(raw: Optional[str] = None) -> str:
    """"disabled", "required" or "auto", from ``raw`` or the environment
    (get_triton_fused_kv_link_mode, pic_runtime.py:1307-1323: same variable,
    aliases, default and error)."""

    mode = (os.getenv("SGLANG_PIC_TRITON_FUSED_KV_LINK", "0") if raw is None else str(raw)).strip().lower()
    normalized = _FUSED_MODE_ALIASES.get(mode)
    if normalized is None:
        raise LinkRuntimeError("SGLANG_PIC_TRITON_FUSED_KV_LINK must be 0, 1, or auto.")
    return normalized


def link_rounding(mode: str, has_clone_blocks: bool) -> tuple[str, Optional[str]]:
    """(rounding, fallback reason) of a link under the fused ``mode``: the
    reference runs its fused kernel only with the mode on and every block read
    from pool slots (pic_runtime.py:5033-5035), else its torch path; "required"
    fails where the fused kernel cannot run (:5153-5157)."""

    if mode == "disabled":
        return "eager", None
    if has_clone_blocks:
        if mode == "required":
            raise LinkRuntimeError("Required Triton LegoLink fusion is unavailable: reference_storage_required")
        return "eager", "reference_storage_required"
    return "fused", None


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

    def set_kv_buffer(self, layer: Any, loc: torch.Tensor, cache_k: torch.Tensor, cache_v: torch.Tensor,
                      k_scale: Optional[float] = None, v_scale: Optional[float] = None) -> None:
        """K_l[loc[i]] = cache_k[i], V likewise, for ``layer.layer_id`` (the
        pool's write of SGLang's MHATokenToKVPool, with its signature): rows of
        another dtype are divided by the layer's scale, when it has one, and
        cast to the pool's.  One ll_kv_scatter_rows launch on the current stream."""

        layer_id = int(getattr(layer, "layer_id", layer))
        key_buffer, value_buffer = self.get_key_buffer(layer_id), self.get_value_buffer(layer_id)

        def stored(rows: torch.Tensor, buffer: torch.Tensor, scale: Optional[float]) -> torch.Tensor:
            rows = rows.reshape(-1, *buffer.shape[1:])
            if rows.dtype != buffer.dtype:
                if scale is not None:
                    rows = rows / scale
                rows = rows.to(buffer.dtype)
            return rows.contiguous().unsqueeze(0)

        kv_link.scatter_kv_rows_inplace(key_buffers=[key_buffer], value_buffers=[value_buffer],
                                        destination_slots=loc, repaired_keys=stored(cache_k, key_buffer, k_scale),
                                        repaired_values=stored(cache_v, value_buffer, v_scale))


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
    """A link's blocks in plan order (pic_runtime.py:4905-5013): everything the
    map builder needs, with no per-token host arrays.  The per-token views
    below (concatenated in plan order) are for inspection and accounting.

    A batch of requests is their blocks request after request, with the
    requests' slots concatenated (``blocks.destination_bases``); repair
    positions are then destination indices."""

    request_slots: torch.Tensor       # the request's slots by request position (on the pool device)
    blocks: link_maps.BlockTable
    handles: list[LegoLinkBlockHandle]
    repair_positions: np.ndarray      # int64, sorted unique imp_indices (destination indices)
    prefix_token_count: int           # identity tokens (block 0 of each request when it needs no remap)
    max_position: int                 # largest local or global position of the link
    leading_blocks: Optional[np.ndarray] = None  # bool [B]: identity blocks
    request_count: int = 1
    block_requests: Optional[np.ndarray] = None  # int64 [B] request of every block (None: one request)

    @classmethod
    def batch(cls, maps: Sequence["LinkMaps"]) -> "LinkMaps":
        """Several requests' links as one."""

        if len(maps) == 1:
            return maps[0]
        sizes = [int(m.request_slots.numel()) for m in maps]
        bases = np.concatenate(([0], np.cumsum(sizes)[:-1])).astype(np.int64)
        request_slots = torch.cat([m.request_slots.to(torch.int64) for m in maps])
        blocks = link_maps.concatenate_tables([m.blocks for m in maps], bases)
        leading = np.concatenate([m.leading_blocks if m.leading_blocks is not None
                                  else np.zeros(m.blocks.counts.size, dtype=bool) for m in maps])
        repair = np.concatenate([m.repair_positions + base for m, base in zip(maps, bases)])
        block_requests, first = [], 0
        for m in maps:
            own = m.block_requests if m.block_requests is not None else np.zeros(m.blocks.counts.size, np.int64)
            block_requests.append(own + first)
            first += m.request_count
        return cls(request_slots=request_slots, blocks=blocks,
                   handles=[h for m in maps for h in m.handles], repair_positions=repair.astype(np.int64),
                   prefix_token_count=sum(m.prefix_token_count for m in maps),
                   max_position=max(m.max_position for m in maps), leading_blocks=leading,
                   request_count=sum(m.request_count for m in maps),
                   block_requests=np.concatenate(block_requests).astype(np.int64))

    def request_has_clone(self) -> np.ndarray:
        """bool [requests]: the request holds a block stored in clone mode."""

        clone = self.blocks.sets == 1
        if self.block_requests is None or self.request_count == 1:
            return np.array([bool(clone.any())])
        return np.bincount(self.block_requests, weights=clone, minlength=self.request_count) > 0

    @property
    def token_count(self) -> int:
        return self.blocks.token_count

    @property
    def local_positions(self) -> np.ndarray:
        return np.concatenate([np.asarray(h.compile_local_positions, dtype=np.int64) for h in self.handles])

    @property
    def global_positions(self) -> np.ndarray:
        return np.concatenate([np.arange(s, s + n, dtype=np.int64)
                               for s, n in zip(self.blocks.starts.tolist(), self.blocks.counts.tolist())])

    @property
    def source_slots(self) -> torch.Tensor:
        return torch.cat([h.slots_on(self.request_slots.device) for h in self.handles])

    @property
    def destination_slots(self) -> torch.Tensor:
        return torch.cat([self.request_slots[s : s + n] for s, n in
                          zip(self.blocks.destination_starts.tolist(), self.blocks.counts.tolist())]).long()

    @property
    def repair_offsets(self) -> np.ndarray:
        """Concatenation offsets of the repair rows inside blocks, in plan order."""

        block, offset = link_maps.repair_rows_in_blocks(self.blocks, self.repair_positions)
        return (self.blocks.offsets[block] + offset).astype(np.int64)

    @property
    def clone_tokens(self) -> np.ndarray:
        return np.repeat(self.blocks.sets == 1, self.blocks.counts)

    @property
    def block_specs(self) -> list[dict[str, Any]]:
        block, _ = link_maps.repair_rows_in_blocks(self.blocks, self.repair_positions)
        repairs = np.bincount(block, minlength=len(self.handles)) if block.size else np.zeros(len(self.handles), int)
        specs = []
        for index, handle in enumerate(self.handles):
            start, count = int(self.blocks.starts[index]), int(self.blocks.counts[index])
            specs.append({
                "block_index": index,
                "cache_key": handle.cache_key,
                "start": start,
                "end": start + count,
                "token_count": count,
                "storage_mode": handle.storage_mode,
                "needs_rope_remap": _needs_rope_remap(handle, start),
                "repair_token_count": int(repairs[index]),
            })
        return specs


_RANGE_FIELDS = operator.itemgetter("start_token", "end_token")


def _range_bounds(ranges: Sequence[Mapping[str, Any]]) -> np.ndarray:
    """int64 ``[B, 2]`` (start_token, end_token) of the plan's block ranges."""

    bounds = np.empty((len(ranges), 2), dtype=np.int64)
    try:
        _host_sequences.fields_from_mappings(ranges, "start_token", "end_token", bounds)
    except (TypeError, OverflowError):  # fields that are not integers: int() of each, as the reference
        bounds = np.array([int(value) for r in ranges for value in _RANGE_FIELDS(r)],
                          dtype=np.int64).reshape(-1, 2)
    return bounds


def _index_array(values: Any) -> np.ndarray:
    """imp_indices as a flat int64 array: a Python list (the reference's plan
    format) or other iterable of integers read item by item in C; arrays and
    tensors as they are."""

    if values is None:
        return np.zeros(0, dtype=np.int64)
    if isinstance(values, torch.Tensor):
        return values.detach().reshape(-1).to("cpu", torch.int64).numpy()
    if isinstance(values, np.ndarray):
        return values.astype(np.int64, copy=False).reshape(-1)
    try:
        if not isinstance(values, (list, tuple)):
            values = list(values)  # any other iterable of integers
        out = np.empty(len(values), dtype=np.int64)
        _host_sequences.int64_from_sequence(values, out)
        return out
    except (TypeError, OverflowError):  # entries that are not integers, or not a sequence
        return np.asarray(values, dtype=np.int64).reshape(-1)


def _needs_rope_remap(handle: LegoLinkBlockHandle, start: int) -> bool:
    """True unless every compile-time position equals the token's global one
    (pic_runtime.py:4951-4955 decides by ``start != 0`` for positions 0..n-1)."""

    if handle.local_start is not None:
        return handle.local_start != start
    return not np.array_equal(np.asarray(handle.compile_local_positions, dtype=np.int64),
                              np.arange(start, start + handle.token_count, dtype=np.int64))


# MI355X's memory-side cache (Infinity Cache): source rows beyond this size
# cannot all be resident, so reading them with non-temporal loads loses nothing.
MEMORY_SIDE_CACHE_BYTES = 256 * 1024 * 1024


def _slot_bytes(buffer: torch.Tensor) -> int:
    """Bytes of one slot's row of a [slots, heads, dim] buffer."""

    return int(buffer.shape[1]) * int(buffer.shape[2]) * buffer.element_size()


def _row_bytes(pool: Any, layer: int) -> int:
    """Bytes of one slot's K row plus V row in ``layer`` of ``pool``."""

    key, value = pool.get_key_buffer(layer), pool.get_value_buffer(layer)
    return int(key[0].numel()) * key.element_size() + int(value[0].numel()) * value.element_size()


def _validate_pool(pool: Any) -> None:
    """pic_runtime.py:6283-6289."""

    if not all(hasattr(pool, method) for method in ("get_key_buffer", "get_value_buffer")):
        raise LinkRuntimeError("PIC link requires an MHA-style KV pool.")
    if getattr(pool, "store_dtype", None) != getattr(pool, "dtype", None):
        raise LinkRuntimeError("PIC link does not yet support quantized KV cache.")


VISIT_ORDERS = ("plan", "source", "destination")


def _resolve_visit_order(visit_order: Optional[str], order_by_source: Optional[bool], request_count: int) -> str:
    """The rows' visit order: ``visit_order`` if given, else "source" /
    "plan" from the older ``order_by_source`` flag, else "source" for a batch
    of requests and "destination" for one."""

    if visit_order is not None:
        if visit_order not in VISIT_ORDERS:
            raise ValueError(f"visit_order must be one of {VISIT_ORDERS}, got {visit_order!r}")
        return visit_order
    if order_by_source is not None:
        return "source" if order_by_source else "plan"
    return "source" if request_count > 1 else "destination"


class PreparedLink:
    """One link, validated and with its device maps built; ``launch()`` enqueues
    the link kernel(s) on the current stream, ``write_repaired()`` the
    repaired-row write-back of the rows the link skipped.

    The maps are written by the map builder on the current stream at
    construction; launch on the same stream (or synchronise first)."""

    def __init__(self, *, pool: Any, layers: list[int], maps: LinkMaps,
                 groups: list[tuple[list[int], RotarySpec]], boundary_repair_aware: bool,
                 compact_repair_rows: bool, num_warps: Optional[int], layers_per_wave: int,
                 validate_indices: bool, arena: Optional[SnapshotArena] = None,
                 layer_groups_per_block: int = 0, order_by_source: Optional[bool] = None,
                 fused_mode: str = "required", delta_staging: str = "auto",
                 skipped_rows: Optional[torch.Tensor] = None, visit_order: Optional[str] = None,
                 order_workspace: Optional[torch.Tensor] = None) -> None:
        self.pool = pool
        self.layers = layers
        self.maps = maps
        self.host_prepare_s = 0.0
        self.boundary_repair_aware = boundary_repair_aware
        key_buffers = [pool.get_key_buffer(layer) for layer in layers]
        value_buffers = [pool.get_value_buffer(layer) for layer in layers]
        self.key_buffers, self.value_buffers = key_buffers, value_buffers
        token_count = maps.token_count
        has_clone = bool((maps.blocks.sets == 1).any())
        if has_clone and arena is None:
            raise LinkRuntimeError("PIC link of clone-mode blocks needs the snapshot arena.")
        self.fused_mode = fused_mode
        # Rounding per request, as the reference decides it per link
        # (pic_runtime.py:5033-5035): a request holding a clone block takes the
        # torch path's rounding, the others the fused kernel's.
        request_clone = maps.request_has_clone()
        decided = [link_rounding(fused_mode, bool(clone)) for clone in request_clone]
        self.request_roundings = [rounding for rounding, _ in decided]
        self.fallback_reason = next((reason for _, reason in decided if reason), None)
        distinct = set(self.request_roundings)
        self.rounding = distinct.pop() if len(distinct) == 1 else "mixed"
        repair_positions = maps.repair_positions if boundary_repair_aware else np.zeros(0, dtype=np.int64)
        plan = link_maps.plan_segments(maps.blocks, repair_positions, compact=compact_repair_rows,
                                       leading_blocks=maps.leading_blocks)
        self.segment_plan = plan
        self.repair_offsets = plan.repair_offsets
        built = link_maps.build_device_maps(plan, maps.request_slots, compact=compact_repair_rows)
        self.device_maps = built
        self.repair_destination_slots = built.repair_destination_slots
        self.linked_token_count = token_count - plan.repair_count
        self._links: list[kv_link.PreparedKVLink] = []
        self._kernel_maps: list[torch.Tensor] = []
        index_of = {layer: i for i, layer in enumerate(layers)}
        # The order in which the kernel visits the rotated rows.  The link's
        # result does not depend on it (every destination is written once);
        # the identity rows stay first, and `device_maps` keeps plan order.
        # A batch of requests often reads the same catalogue blocks: in
        # source-slot order, repeated sources are read close together and hit
        # in cache (c3: 6.2 -> 7.2 TB/s; destination order 6.3-6.4).  A single
        # request reads each row once, and its scattered writes cost more than
        # its scattered reads: in destination-slot order c2's link runs 1.8 %
        # faster (0.7465 -> 0.7334 ms), c4's 1.0 % and c5's 2.4 %.
        self.visit_order = _resolve_visit_order(visit_order, order_by_source, maps.request_count)
        self.order_by_source = self.visit_order == "source"
        # A single request reads each source row about once: when its rows are
        # larger than the memory-side cache, non-temporal row loads keep them
        # out of the caches (c2 +2 %, c5 +8 %).  Batched requests share
        # catalogue blocks, whose repeated rows should hit in cache, and rows
        # that fit the memory-side cache may already be there.
        key_row = _slot_bytes(key_buffers[0])
        value_row = _slot_bytes(value_buffers[0])
        row_bytes = key_row + value_row
        self.stream_source_rows = (maps.request_count == 1 and not self.order_by_source
                                   and token_count * len(layers) * row_bytes > MEMORY_SIDE_CACHE_BYTES)
        sort_row = {"source": 0, "destination": 1}.get(self.visit_order)
        if sort_row == 1 and order_workspace is None:
            order_workspace = torch.zeros(_native.ORDER_WORKSPACE_BYTES, dtype=torch.uint8,
                                          device=key_buffers[0].device)
        # delta_staging "table": a layer-major value pass writes every token's
        # RoPE delta to a table and a layer-major key pass reads it back
        # (measured 1.4-2.0 % slower than the default staged deltas on c2,
        # c4, c5); the launches run one after another on one stream and share
        # one workspace.
        self.delta_workspace = None
        if (delta_staging == "table"
                and int(key_buffers[0].shape[1]) * int(key_buffers[0].shape[2]) % 512 == 0):
            widest = max(int(rotary.rotary_dim) for _, rotary in groups)
            counts = [plan.map_counts[s] for s in (0, 1)]
            self.delta_workspace = torch.empty(kv_link.delta_workspace_bytes(max(counts), widest),
                                               dtype=torch.uint8, device=key_buffers[0].device)
        # Under a mixed batch, the pool set's entries of clone-holding requests
        # are eager, the others fused; the snapshot arena's are always eager.
        request_eager = np.array([rounding == "eager" for rounding in self.request_roundings])
        # One launch per source (set 0 reads the pool, set 1 the snapshot arena),
        # per rounding within it.
        for source_set in (0, 1):
            device_maps = built.maps[source_set]
            if device_maps is None:
                continue
            source_arena = arena if source_set == 1 else None
            prefix = plan.set_prefix[source_set]
            mask = built.masks[source_set] if plan.set_repair_rows[source_set] else None
            count = int(device_maps.shape[1])
            eager_entries = None
            if self.rounding != "mixed":
                pieces = [(0, count, self.rounding, prefix)]
            elif source_set == 1:
                pieces = [(0, count, "eager", prefix)]
            else:
                run_eager = request_eager[maps.block_requests[plan.segment_blocks]]
                eager_entries = link_maps.set_entry_flags(plan, 0, run_eager, compact=compact_repair_rows)
                # Identity entries are bit copies in either rounding: they stay
                # at the head, with the fused entries after them.
                split = prefix + int(np.count_nonzero(eager_entries[prefix:] == 0))
                pieces = [(0, split, "fused", prefix), (split, count, "eager", 0)]
            if sort_row == 1 and eager_entries is None and count - prefix > 1:
                # Destination order by the library's bucketed counting sort
                # (three launches, where torch's argsort takes about ten).
                # Source order stays an exact sort: a batch's repeated source
                # rows must be adjacent to hit in cache (bucketed, c3's link
                # ran 2.7-3.6 % slower: 8.59-8.65 against 8.35-8.39 ms).
                device_maps, mask = link_maps.order_link_maps(
                    device_maps, mask.view(torch.uint8) if mask is not None else None, key_row=1,
                    prefix=prefix, num_slots=int(key_buffers[0].shape[0]), workspace=order_workspace)
                self._kernel_maps.append(device_maps)
            elif (sort_row is not None or eager_entries is not None) and count - prefix > 1:
                tail = device_maps[:, prefix:]
                key = None if sort_row is None else tail[sort_row]
                if eager_entries is not None:
                    # The rounding class first (slots below 2^40 keep their order within it).
                    group = torch.from_numpy(eager_entries[prefix:].astype(np.int64)).to(device_maps.device) << 40
                    key = group if key is None else key.clamp(0, (1 << 40) - 1) + group
                order = torch.argsort(key, stable=True)
                device_maps = tail[:, order] if prefix == 0 else torch.cat([device_maps[:, :prefix], tail[:, order]],
                                                                              dim=1)
                if mask is not None:
                    mask = mask[prefix:][order] if prefix == 0 else torch.cat([mask[:prefix], mask[prefix:][order]])
                self._kernel_maps.append(device_maps)
            for begin, end, rounding, piece_prefix in pieces:
                if end <= begin:
                    continue
                for group_index, (group_layers, rotary) in enumerate(groups):
                    indices = [index_of[layer] for layer in group_layers]
                    self._links.append(kv_link.PreparedKVLink(
                        key_buffers=[key_buffers[i] for i in indices],
                        value_buffers=[value_buffers[i] for i in indices],
                        source_slots=device_maps[0, begin:end],
                        destination_slots=device_maps[1, begin:end],
                        local_positions=device_maps[2, begin:end],
                        global_positions=device_maps[3, begin:end],
                        cos_sin_cache=rotary.cos_sin_cache,
                        prefix_token_count=min(piece_prefix, end - begin),
                        rotary_dim=rotary.rotary_dim,
                        is_neox_style=rotary.is_neox_style,
                        repair_mask=None if mask is None else mask[begin:end],
                        num_warps=num_warps,
                        layers_per_wave=layers_per_wave,
                        layer_groups_per_block=layer_groups_per_block,
                        validate_indices=validate_indices,
                        source_key_buffers=(None if source_arena is None else
                                            [source_arena.get_key_buffer(layer) for layer in group_layers]),
                        source_value_buffers=(None if source_arena is None else
                                              [source_arena.get_value_buffer(layer) for layer in group_layers]),
                        stream_source_rows=self.stream_source_rows,
                        rounding=rounding,
                        delta_staging=delta_staging,
                        # Each launch's tokens are counted once, by its first layer group.
                        skipped_rows=skipped_rows if group_index == 0 else None,
                        delta_workspace=self.delta_workspace,
                    ))
        self.traffic = kv_link.estimate_kv_traffic_bytes(
            token_count=token_count,
            key_row_bytes=key_row,
            value_row_bytes=value_row,
            remapped_token_count=token_count - maps.prefix_token_count,
            repair_token_count=plan.repair_count,
        )
        self.algorithmic_link_bytes = self.linked_token_count * (key_row + value_row) * 2 * len(layers)

    @property
    def kernel_maps(self) -> list[torch.Tensor]:
        """The device maps the link kernels read, one [4, N] int64 tensor per
        source (source slot, destination slot, local and global position per
        token, in the visit order)."""

        return list(self._kernel_maps)

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
        blocks = self.maps.blocks
        return {
            "token_count": self.maps.token_count,
            "linked_token_count": self.linked_token_count,
            "block_count": len(self.maps.handles),
            "prefix_token_count": self.maps.prefix_token_count,
            "remapped_token_count": self.maps.token_count - self.maps.prefix_token_count,
            "repair_token_count": int(self.repair_offsets.size),
            "boundary_repair_aware": self.boundary_repair_aware,
            "layers_written": len(self.layers),
            "kernel_launches": sum(info["launches"] for info in self.launch_info),
            "launch": self.launch_info,
            "rope_remapped": [_needs_rope_remap(handle, start)
                              for handle, start in zip(self.maps.handles, blocks.starts.tolist())],
            "storage_modes": [handle.storage_mode for handle in self.maps.handles],
            "map_runs": int(self.segment_plan.table.shape[0]),
            "fused_mode": self.fused_mode,
            "rounding": self.rounding,
            "request_roundings": list(self.request_roundings),
            "fallback_reason": self.fallback_reason,
            **self.traffic,
        }


class KVLinkExecutor:
    """Links registered blocks into request slots on one GPU."""

    def __init__(self, registry: LegoLinkBlockRegistry, rotary: Any, *,
                 start_layer: int = 0, end_layer: int, num_warps: Optional[int] = None,
                 layers_per_wave: int = 0, arena: Optional[SnapshotArena] = None,
                 layer_groups_per_block: int = 0, fused_mode: Optional[str] = None,
                 delta_staging: str = "auto", count_skipped_rows: bool = True,
                 visit_order: Optional[str] = None) -> None:
        """``rotary`` is a RotarySpec, a model's rotary module, or a mapping of
        layer to either.  ``fused_mode`` ("disabled" / "required" / "auto", or the reference's
        aliases) fixes the link's rounding; None reads
        ``SGLANG_PIC_TRITON_FUSED_KV_LINK`` at every link, as the reference does.
        ``delta_staging`` ("auto" / "per_wave" / "workgroup") picks where the
        link kernel computes its RoPE deltas (the result is the same).
        ``count_skipped_rows`` has every link count, on the device, the
        tokens its kernel skipped for an out-of-range slot or position
        (``skipped_rows`` / ``check_skipped_rows`` read the count)."""

        if visit_order is not None and visit_order not in VISIT_ORDERS:
            raise ValueError(f"visit_order must be one of {VISIT_ORDERS}, got {visit_order!r}")
        self.visit_order = visit_order
        self.registry = registry
        self.fused_mode = None if fused_mode is None else get_fused_kv_link_mode(fused_mode)
        self.delta_staging = delta_staging
        self.start_layer = int(start_layer)
        self.end_layer = int(end_layer)
        # A model's rotary module (sglang's RotaryEmbedding and the like) is
        # wrapped once, so layers sharing a module share one spec.
        wrapped: dict[int, RotarySpec] = {}

        def spec_of(value: Any) -> RotarySpec:
            if isinstance(value, RotarySpec):
                return value
            if id(value) not in wrapped:
                wrapped[id(value)] = RotarySpec.from_module(value)
            return wrapped[id(value)]

        if isinstance(rotary, Mapping):
            self.rotary_by_layer = {int(layer): spec_of(value) for layer, value in rotary.items()}
        else:
            spec = spec_of(rotary)
            self.rotary_by_layer = {layer: spec for layer in range(self.start_layer, self.end_layer)}
        self.num_warps = num_warps
        self.layers_per_wave = layers_per_wave
        self.layer_groups_per_block = layer_groups_per_block
        self.arena = arena
        self.count_skipped_rows = bool(count_skipped_rows)
        self._skip_counters: dict[torch.device, torch.Tensor] = {}
        self._order_workspaces: dict[torch.device, torch.Tensor] = {}

    @property
    def layers(self) -> list[int]:
        return list(range(self.start_layer, self.end_layer))

    def _skip_counter(self, device: torch.device) -> Optional[torch.Tensor]:
        if not self.count_skipped_rows:
            return None
        device = torch.device(device)
        counter = self._skip_counters.get(device)
        if counter is None:
            counter = torch.zeros(1, dtype=torch.int64, device=device)
            self._skip_counters[device] = counter
        return counter

    def _order_workspace(self, device: torch.device) -> torch.Tensor:
        """The zeroed workspace of the destination ordering on ``device``,
        shared by this executor's links (prepared on one stream)."""

        device = torch.device(device)
        workspace = self._order_workspaces.get(device)
        if workspace is None:
            workspace = torch.zeros(_native.ORDER_WORKSPACE_BYTES, dtype=torch.uint8, device=device)
            self._order_workspaces[device] = workspace
        return workspace

    def skipped_rows(self, *, reset: bool = True) -> int:
        """Tokens the links so far skipped because a slot or position was out
        of range (the kernels skip such rows; the reference's eager path raises
        on them).  Reads the device counters, which waits for the work already
        queued on the current stream; links launched on other streams must be
        synchronised first.  ``reset`` zeroes the counters."""

        total = 0
        for counter in self._skip_counters.values():
            total += int(counter.item())
            if reset:
                counter.zero_()
        return total

    def check_skipped_rows(self) -> None:
        """Raise if any link since the last check skipped a token."""

        skipped = self.skipped_rows(reset=True)
        if skipped:
            raise LinkRuntimeError(f"PIC link skipped {skipped} token(s): a slot or RoPE position was out of range.")

    def _fused_mode(self) -> str:
        return self.fused_mode if self.fused_mode is not None else get_fused_kv_link_mode()

    # -- maps ---------------------------------------------------------------
    def build_link_maps(self, destination_slots: torch.Tensor, link_plan: Mapping[str, Any],
                        *, device: Optional[torch.device] = None) -> LinkMaps:
        """The plan's blocks in plan order (pic_runtime.py:4905-5013): lookups and
        checks per block, then block-level arrays for the map builder."""

        ranges = link_plan.get("block_ranges") or link_plan.get("attention_ranges")
        cache_keys = link_plan.get("cache_keys")
        if not isinstance(ranges, list) or not isinstance(cache_keys, list):
            raise LinkRuntimeError("PIC link plan is missing block ranges/cache keys.")
        if len(ranges) != len(cache_keys):
            raise LinkRuntimeError("PIC block range and cache key counts differ.")
        if not cache_keys:
            raise LinkRuntimeError("PIC link plan has no blocks.")
        handles, unavailable = self.registry.link_handles(list(map(str, cache_keys)))
        if unavailable:
            missing = [key for key, handle in zip(cache_keys, handles) if handle is None]
            stale = [key for key, handle in zip(cache_keys, handles) if handle is not None and not handle.valid]
            raise LinkRuntimeError(
                f"PIC RadixCache lookup cannot safely link block(s): {', '.join(map(str, missing + stale))}"
            )
        device = destination_slots.device if device is None else device
        request_slots = destination_slots
        if request_slots.device != device or request_slots.dtype not in (torch.int32, torch.int64):
            request_slots = request_slots.to(device=device, dtype=torch.int64)
        request_slots = request_slots.contiguous()
        total = int(request_slots.numel())
        # Per block: the handle's cached record (count, slot and position
        # addresses, local start, set, max local position) and the plan range.
        records = self.registry.link_records(handles, device)
        bounds = _range_bounds(ranges)
        starts, ends = bounds[:, 0].copy(), bounds[:, 1]
        counts = records[:, 0].copy()
        mismatch = np.flatnonzero(ends - starts != counts)
        if mismatch.size:
            index = int(mismatch[0])
            raise LinkRuntimeError(
                f"PIC token count mismatch for block {handles[index].cache_key}: "
                f"plan={int(ends[index] - starts[index])}, snapshot={int(counts[index])}"
            )
        outside = np.flatnonzero((ends > total) | (starts < 0))
        if outside.size:
            raise LinkRuntimeError(
                f"PIC block {handles[int(outside[0])].cache_key} range exceeds the request's slots.")
        source_ptrs = records[:, 1].copy()
        local_ptrs = records[:, 2].copy()
        local_starts = records[:, 3].copy()
        sets = records[:, 4].copy()
        max_position = int(max(int(ends.max()) - 1, int(records[:, 5].max())))
        blocks = link_maps.BlockTable(starts=starts, counts=counts, source_ptrs=source_ptrs,
                                      local_ptrs=local_ptrs, local_starts=local_starts, sets=sets)
        # Sorted or not, duplicates allowed: the run planner sorts and dedups.
        repair = _index_array(link_plan.get("imp_indices"))
        identity = not _needs_rope_remap(handles[0], int(starts[0]))
        leading = np.zeros(len(handles), dtype=bool)
        leading[0] = identity
        return LinkMaps(request_slots=request_slots, blocks=blocks, handles=handles,
                        repair_positions=repair, prefix_token_count=int(counts[0]) if identity else 0,
                        max_position=int(max_position), leading_blocks=leading)

    def build_batch_link_maps(self, requests: Sequence[tuple[torch.Tensor, Mapping[str, Any]]],
                              *, device: torch.device) -> LinkMaps:
        """``LinkMaps.batch`` of every request's ``build_link_maps``, with one
        registry lookup, one record gather and vectorised range checks for the
        whole batch.  A batch with any fault is rebuilt request by request, so
        the error raised is the one that request's own link raises."""

        def one_by_one() -> LinkMaps:
            return LinkMaps.batch([self.build_link_maps(slots, plan, device=device) for slots, plan in requests])

        if not requests:
            raise LinkRuntimeError("PIC batched link has no requests.")
        if len(requests) == 1:
            return one_by_one()
        range_lists, key_lists, repair_lists = [], [], []
        for _, plan in requests:
            ranges = plan.get("block_ranges") or plan.get("attention_ranges")
            cache_keys = plan.get("cache_keys")
            if (not isinstance(ranges, list) or not isinstance(cache_keys, list)
                    or len(ranges) != len(cache_keys) or not cache_keys):
                return one_by_one()
            range_lists.append(ranges)
            key_lists.append(cache_keys)
            repair_lists.append(plan.get("imp_indices"))
        block_counts = np.fromiter(map(len, key_lists), dtype=np.int64, count=len(key_lists))
        handles, unavailable = self.registry.link_handles(
            list(map(str, itertools.chain.from_iterable(key_lists))))
        if unavailable:
            return one_by_one()
        slot_tensors = [slots if slots.device == device and slots.dtype == torch.int64
                        else slots.to(device=device, dtype=torch.int64) for slots, _ in requests]
        sizes = np.fromiter((int(slots.numel()) for slots in slot_tensors), dtype=np.int64, count=len(requests))
        bases = link_maps.exclusive_offsets(sizes)
        records = self.registry.link_records(handles, device)
        bounds = _range_bounds(list(itertools.chain.from_iterable(range_lists)))
        starts, ends = bounds[:, 0].copy(), bounds[:, 1]
        counts = records[:, 0].copy()
        totals = np.repeat(sizes, block_counts)
        if ((ends - starts != counts) | (ends > totals) | (starts < 0)).any():
            return one_by_one()
        firsts = link_maps.exclusive_offsets(block_counts)
        leading = np.zeros(len(handles), dtype=bool)
        leading[firsts] = [not _needs_rope_remap(handles[first], start)
                           for first, start in zip(firsts.tolist(), starts[firsts].tolist())]
        blocks = link_maps.BlockTable(starts=starts, counts=counts, source_ptrs=records[:, 1].copy(),
                                      local_ptrs=records[:, 2].copy(), local_starts=records[:, 3].copy(),
                                      sets=records[:, 4].copy(), destination_bases=np.repeat(bases, block_counts))
        # Per request, the largest position is max(end - 1, largest local
        # position); over the batch that is the maximum of both columns.
        max_position = int(max(int(ends.max()) - 1, int(records[:, 5].max())))
        repair_lists = [[] if values is None else values for values in repair_lists]
        if all(type(values) is list for values in repair_lists):
            # The reference's plan format: one conversion of every request's
            # list, then each request's base added.
            lengths = np.fromiter(map(len, repair_lists), dtype=np.int64, count=len(repair_lists))
            repair = _index_array(list(itertools.chain.from_iterable(repair_lists))) + np.repeat(bases, lengths)
        else:
            repair = np.concatenate([_index_array(values) + base
                                     for values, base in zip(repair_lists, bases.tolist())]).astype(np.int64)
        return LinkMaps(request_slots=torch.cat(slot_tensors), blocks=blocks, handles=handles,
                        repair_positions=repair, prefix_token_count=int(counts[leading].sum()),
                        max_position=max_position, leading_blocks=leading, request_count=len(requests),
                        block_requests=np.repeat(np.arange(len(requests), dtype=np.int64), block_counts))

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
        groups = self._layer_groups(self.layers, maps.max_position, device)
        prepared = PreparedLink(
            pool=pool, layers=self.layers, maps=maps, groups=groups,
            boundary_repair_aware=bool(boundary_repair_aware), compact_repair_rows=compact_repair_rows,
            num_warps=self.num_warps, layers_per_wave=self.layers_per_wave,
            validate_indices=validate_indices, arena=self.arena,
            layer_groups_per_block=self.layer_groups_per_block, fused_mode=self._fused_mode(),
            delta_staging=self.delta_staging, skipped_rows=self._skip_counter(device),
            visit_order=self.visit_order, order_workspace=self._order_workspace(device),
        )
        prepared.host_prepare_s = time.perf_counter() - started
        return prepared

    def prepare_links(self, pool: Any, requests: Sequence[tuple[torch.Tensor, Mapping[str, Any]]], *,
                      boundary_repair_aware: Optional[bool] = None, compact_repair_rows: bool = True,
                      validate_indices: bool = False, order_by_source: Optional[bool] = None) -> PreparedLink:
        """Several requests' links as one prepared link: one map-builder call and
        one link launch per source for the whole batch.  ``requests`` holds
        (destination_slots, link_plan) pairs; the result equals linking them one
        by one (destinations of different requests must be distinct).  Every
        request's identity block heads its set's maps, so it is copied
        unrotated as in a single link; the repair rows of the write-back are
        request after request, each in plan order.  ``order_by_source``
        (default: on for more than one request) has the kernel visit the
        rotated rows in source-slot order."""

        started = time.perf_counter()
        if not requests:
            raise LinkRuntimeError("PIC batched link has no requests.")
        _validate_pool(pool)
        if boundary_repair_aware is None:
            boundary_repair_aware = _env_flag("SGLANG_PIC_TRITON_BOUNDARY_REPAIR_AWARE", "0")
        device = pool.get_key_buffer(self.start_layer).device
        maps = self.build_batch_link_maps(requests, device=device)
        groups = self._layer_groups(self.layers, maps.max_position, device)
        prepared = PreparedLink(
            pool=pool, layers=self.layers, maps=maps, groups=groups,
            boundary_repair_aware=bool(boundary_repair_aware), compact_repair_rows=compact_repair_rows,
            num_warps=self.num_warps, layers_per_wave=self.layers_per_wave,
            validate_indices=validate_indices, arena=self.arena,
            layer_groups_per_block=self.layer_groups_per_block, order_by_source=order_by_source,
            fused_mode=self._fused_mode(), delta_staging=self.delta_staging,
            skipped_rows=self._skip_counter(device),
            visit_order=None if order_by_source is not None else self.visit_order,
            order_workspace=self._order_workspace(device),
        )
        prepared.host_prepare_s = time.perf_counter() - started
        return prepared

    def copy_linked_kv(self, pool: Any, destination_slots: torch.Tensor, link_plan: Mapping[str, Any],
                       *, raise_on_skip: bool = False, **options: Any) -> dict[str, Any]:
        """Link the plan's blocks into ``destination_slots`` (the request's slots
        indexed by request position) on the current stream; returns an
        accounting record.  Blocks stay pinned while the link is enqueued.

        The kernel skips a token whose slot or RoPE position is out of range
        and counts it on the device, where the reference's torch path raises.
        ``raise_on_skip`` reads the count after the launch (which waits for the
        stream) and raises ``LinkRuntimeError`` if any token was skipped;
        without it the caller polls ``check_skipped_rows()``."""

        lookup = self.registry.lookup_legolink_blocks(str(key) for key in link_plan.get("cache_keys") or [])
        handles = self.registry.acquire_legolink_blocks(lookup.matched_handles)
        try:
            prepared = self.prepare_link(pool, destination_slots, link_plan, **options)
            prepared.launch()
        finally:
            self.registry.release_legolink_blocks(handles)
        if raise_on_skip:
            self.check_skipped_rows()
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
    def _copy_rows(self, *, destination: Any, source: Any, source_slots: torch.Tensor,
                   destination_slots: torch.Tensor, local: torch.Tensor, global_: torch.Tensor,
                   prefix: int, rounding: str = "fused") -> None:
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
                stream_source_rows=(int(source_slots.numel()) * len(group_layers)
                                    * _row_bytes(source, group_layers[0]) > MEMORY_SIDE_CACHE_BYTES),
                rounding=rounding,
                skipped_rows=self._skip_counter(source_slots.device) if group_layers is groups[0][0] else None,
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

    def capture_blocks(self, pool: Any, blocks: Sequence[Mapping[str, Any]]) -> list[LegoLinkBlockHandle]:
        """Register several compiled blocks at once, as capture_compile_blocks does
        for every compile request of a forward batch (pic_runtime.py:3485-3560).
        Each entry holds ``cache_key``, ``token_ids``, ``slots`` and optionally
        ``storage_mode`` ("reference" or "clone"), ``compile_local_positions`` and
        ``block_id``.
        The clone blocks' rows are copied into their arena ranges by one launch
        over every layer; on any error no block is registered and no arena range
        is kept."""

        _validate_pool(pool)
        device = pool.get_key_buffer(self.start_layer).device
        entries = []
        for block in blocks:
            mode = block.get("storage_mode", "reference")
            if mode not in ("reference", "clone"):
                raise LinkRuntimeError(f"Unsupported PIC storage mode: {mode}")
            slots = torch.as_tensor(block["slots"]).long().reshape(-1).to(device)
            entries.append((block, mode, slots))
        clones = [entry for entry in entries if entry[1] == "clone"]
        if clones and self.arena is None:
            raise LinkRuntimeError("PIC clone storage needs a snapshot arena.")
        ranges: list[torch.Tensor] = []
        handles: list[LegoLinkBlockHandle] = []
        try:
            for block, _, slots in clones:
                arena_slots = self.arena.alloc(int(slots.numel()))
                if arena_slots is None:
                    raise LinkRuntimeError(f"PIC snapshot arena has no {int(slots.numel())} free slots for "
                                           f"{block['cache_key']}.")
                ranges.append(arena_slots)
            if clones:
                source = torch.cat([slots for _, _, slots in clones])
                target = torch.cat(ranges)
                positions = torch.zeros(int(source.numel()), dtype=torch.long, device=device)
                self._copy_rows(destination=self.arena, source=pool, source_slots=source,
                                destination_slots=target, local=positions, global_=positions,
                                prefix=int(source.numel()))
            arena_of = {id(entry[0]): arena_slots for entry, arena_slots in zip(clones, ranges)}
            for block, mode, slots in entries:
                handles.append(self.registry.register_legolink_block(
                    block["cache_key"], block["token_ids"], arena_of.get(id(block), slots),
                    compile_local_positions=block.get("compile_local_positions"),
                    block_id=block.get("block_id"), storage_mode=mode))
            return handles
        except Exception:
            for handle in handles:
                self.registry.evict_legolink_block(handle.cache_key)
            for arena_slots in ranges:
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
        when the group starts at position 0, with the torch path's rounding
        (``_remap_key_positions``, :5914-5919) whatever the fused mode."""

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
                        prefix=0, rounding="eager")
        return self.registry.register_legolink_block(cache_key, token_ids, new_slots,
                                                     storage_mode="reference")
