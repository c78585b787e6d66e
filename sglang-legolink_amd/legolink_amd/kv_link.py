"""HIP LegoLink KV link operator: gather, RoPE delta re-rotation and scatter.

Drop-in counterpart of ``patched_sglang_files/python/sglang/srt/legolink_triton.py``:
the same public names, keyword arguments, eligibility reasons, exception types
and traffic model, backed by the hand-written gfx950 kernels in
``liblegolink_kv.so`` instead of a Triton JIT kernel.

Two entries go beyond the reference operator:

* ``fused_kv_link_layers_inplace`` links every layer of the pool in one launch
  (the reference calls its operator once per layer, pic_runtime.py:5168-5208);
* ``scatter_kv_rows_inplace`` writes repaired boundary rows into the pool
  (the repair pass's K/V write, flashinfer_sparse_repair.py:2235-2239).

Every tensor stays owned by the caller; nothing here allocates device memory.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Any, Sequence

import torch

from . import _native

# Reason reported when the HIP library cannot be loaded; the reference reports
# "triton_not_installed" in the same position (legolink_triton.py:174-175).
NATIVE_UNAVAILABLE_REASON = "hip_kv_link_not_built"


@dataclass(frozen=True)
class LegoLinkFusionEligibility:
    supported: bool
    reason: str


@dataclass(frozen=True)
class LegoLinkLaunchConfig:
    block_size: int
    num_warps: int
    num_stages: int
    source: str


_KV_DTYPES = {torch.float16: _native.DTYPE_FLOAT16, torch.bfloat16: _native.DTYPE_BFLOAT16}
_CACHE_DTYPES = {
    torch.float16: _native.DTYPE_FLOAT16,
    torch.bfloat16: _native.DTYPE_BFLOAT16,
    torch.float32: _native.DTYPE_FLOAT32,
}
_INDEX_DTYPES = {torch.int32: _native.DTYPE_INT32, torch.int64: _native.DTYPE_INT64}

# Rounding of re-rotated K: "fused" is the reference's fused kernel
# (legolink_triton.py:413-470), "eager" its torch path (pic_runtime.py:6025-6058
# with _apply_rotary_emb, :1868-1885).
ROUNDINGS = {"fused": _native.ROUNDING_FUSED, "eager": _native.ROUNDING_EAGER}


# Where the vector kernel computes each token's RoPE delta (the result is the
# same): "per_wave" (each wave from the table), "workgroup" (once per workgroup
# into LDS, the table rows read once per token), "table" (once per token into
# a workspace by a first launch, then a layer-major second launch reads them;
# needs ``delta_workspace``), "auto" (the library's choice).
DELTA_STAGINGS = {"auto": _native.DELTA_AUTO, "per_wave": _native.DELTA_PER_WAVE,
                  "workgroup": _native.DELTA_WORKGROUP, "table": _native.DELTA_TABLE}


def delta_workspace_bytes(token_count: int, rotary_dim: int) -> int:
    """Bytes of the delta table of a link of ``token_count`` tokens: an fp32
    (dc, ds) per token and rotary pair."""

    return int(token_count) * int(rotary_dim) * 4
_DELTA_NAMES = {code: name for name, code in DELTA_STAGINGS.items()}


def _launch_record(info: _native.LaunchInfo) -> dict[str, Any]:
    return {
        "kernel": "vector" if info.kernel == _native.KERNEL_VECTOR else "generic",
        "launches": int(info.launches),
        "grid_x": int(info.grid_x),
        "grid_y": int(info.grid_y),
        "block_threads": int(info.block_threads),
        "layers_per_wave": int(info.layers_per_wave),
        "layer_groups_per_block": int(info.layer_groups_per_block),
        "delta_staging": _DELTA_NAMES.get(int(info.delta_staging)),
    }


def _rounding_code(rounding: str) -> int:
    try:
        return ROUNDINGS[rounding]
    except KeyError:
        raise ValueError(f"rounding must be one of {sorted(ROUNDINGS)}, got {rounding!r}") from None


def resolve_fused_kv_launch_config(
    *,
    work_items: int,
    device: torch.device | None = None,
    capability: tuple[int, int] | None = None,
    block_size: int | None = None,
    num_warps: int | None = None,
    num_stages: int | None = None,
) -> LegoLinkLaunchConfig:
    """Resolve and validate the launch keywords (legolink_triton.py:38-99).

    Same validation rules, defaults and environment overrides
    (``SGLANG_PIC_TRITON_BLOCK_SIZE`` / ``_NUM_WARPS`` / ``_NUM_STAGES``) as the
    reference.  On gfx950 ``num_warps`` is the number of 64-lane waves per
    workgroup; ``block_size`` and ``num_stages`` are validated and recorded but
    do not shape the HIP kernels (their work unit is a 16-byte row chunk of one
    layer row, and each wave walks a short run of layers).
    """

    del work_items, device, capability  # one gfx950 default for every shape
    defaults = (256, 4, 2)
    source = "gfx950_default"
    env_values = (
        os.getenv("SGLANG_PIC_TRITON_BLOCK_SIZE"),
        os.getenv("SGLANG_PIC_TRITON_NUM_WARPS"),
        os.getenv("SGLANG_PIC_TRITON_NUM_STAGES"),
    )
    explicit_values = (block_size, num_warps, num_stages)
    resolved = []
    overridden = False
    for explicit, environment, default in zip(explicit_values, env_values, defaults, strict=True):
        if explicit is not None:
            resolved.append(int(explicit))
            overridden = True
        elif environment not in (None, ""):
            resolved.append(int(environment))
            overridden = True
        else:
            resolved.append(default)
    if overridden:
        source = "explicit_or_environment_override"
    resolved_block_size, resolved_num_warps, resolved_num_stages = resolved
    if (
        resolved_block_size <= 0
        or resolved_block_size > 1024
        or resolved_block_size & (resolved_block_size - 1)
    ):
        raise ValueError("block_size must be a power of two between 1 and 1024")
    if resolved_num_warps not in (1, 2, 4, 8):
        raise ValueError("num_warps must be one of 1, 2, 4, or 8")
    if not 1 <= resolved_num_stages <= 5:
        raise ValueError("num_stages must be between 1 and 5")
    return LegoLinkLaunchConfig(resolved_block_size, resolved_num_warps, resolved_num_stages, source)


def hip_legolink_available() -> bool:
    """True when the HIP library loads and a ROCm device is visible."""

    return _native.library_available() and torch.cuda.is_available()


# Name kept for callers written against the reference module.
triton_legolink_available = hip_legolink_available


def estimate_kv_traffic_bytes(
    *,
    token_count: int,
    key_row_bytes: int,
    value_row_bytes: int,
    remapped_token_count: int,
    repair_token_count: int = 0,
) -> dict[str, int | float]:
    """Lower-bound HBM traffic of the eager torch path and of the fused link.

    Same model and keys as legolink_triton.py:107-156: the fused link reads and
    writes K and V of every copied (non-repair) token once; position maps and
    the cos/sin table are excluded.
    """

    tokens = max(int(token_count), 0)

    def within(count: int) -> int:
        return max(min(int(count), tokens), 0)

    remapped, repair = within(remapped_token_count), within(repair_token_count)
    k_row, v_row = max(int(key_row_bytes), 0), max(int(value_row_bytes), 0)
    copied = tokens - repair
    # One direction (the reads, and equally the writes).  The eager path
    # gathers K and V into temporaries and copies them back (2 row moves per
    # token) and materialises the remapped K once more; the fused link moves
    # each copied token's K and V row once.
    eager_one_way = 2 * tokens * (k_row + v_row) + remapped * k_row
    fused_one_way = copied * (k_row + v_row)
    eager_total, fused_total = 2 * eager_one_way, 2 * fused_one_way
    return {
        "torch_lower_bound_bytes": eager_total,
        "triton_lower_bound_bytes": fused_total,
        "torch_estimated_hbm_read_bytes": eager_one_way,
        "torch_estimated_hbm_write_bytes": eager_one_way,
        "triton_estimated_hbm_read_bytes": fused_one_way,
        "triton_estimated_hbm_write_bytes": fused_one_way,
        "torch_estimated_hbm_traffic_bytes": eager_total,
        "triton_estimated_hbm_traffic_bytes": fused_total,
        "estimated_reduction_ratio": 1.0 - fused_total / eager_total if eager_total else 0.0,
        "copied_token_count": copied,
        "repair_token_count": repair,
    }


def _eligibility(
    key_buffers: Sequence[torch.Tensor],
    value_buffers: Sequence[torch.Tensor],
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    rotary_dim: int,
    repair_mask: torch.Tensor | None,
    source_key_buffers: Sequence[torch.Tensor] = (),
    source_value_buffers: Sequence[torch.Tensor] = (),
) -> LegoLinkFusionEligibility:
    """The reference's checks in the reference's order (legolink_triton.py:159-247),
    applied to every layer (and to a separate source pool, which must have the
    destination pool's row layout), followed by the checks the raw-pointer
    kernels need."""

    if not _native.library_available():
        return LegoLinkFusionEligibility(False, NATIVE_UNAVAILABLE_REASON)
    key_buffer, value_buffer = key_buffers[0], value_buffers[0]
    if len(source_key_buffers) != len(source_value_buffers) or (
        source_key_buffers and len(source_key_buffers) != len(key_buffers)
    ):
        return LegoLinkFusionEligibility(False, "kv_head_layout_mismatch")
    tensors = (
        *key_buffers,
        *value_buffers,
        *source_key_buffers,
        *source_value_buffers,
        source_slots,
        destination_slots,
        local_positions,
        global_positions,
        cos_sin_cache,
    )
    if not all(tensor.is_cuda for tensor in tensors):
        return LegoLinkFusionEligibility(False, "cuda_tensors_required")
    for key, value in zip(key_buffers, value_buffers, strict=True):
        if key.ndim != 3 or value.ndim != 3:
            return LegoLinkFusionEligibility(False, "mha_3d_kv_buffers_required")
        if key.shape[:2] != value.shape[:2] or key.shape != key_buffer.shape or (
            value.shape != value_buffer.shape
        ):
            return LegoLinkFusionEligibility(False, "kv_head_layout_mismatch")
        if key.dtype != value.dtype or key.dtype != key_buffer.dtype:
            return LegoLinkFusionEligibility(False, "kv_dtype_mismatch")
    if source_key_buffers:
        source_rows = int(source_key_buffers[0].shape[0]) if source_key_buffers[0].ndim == 3 else -1
        for key, value in zip(source_key_buffers, source_value_buffers, strict=True):
            if key.ndim != 3 or value.ndim != 3:
                return LegoLinkFusionEligibility(False, "mha_3d_kv_buffers_required")
            if key.shape[1:] != key_buffer.shape[1:] or value.shape[1:] != value_buffer.shape[1:] or (
                int(key.shape[0]) != source_rows or int(value.shape[0]) != source_rows
            ):
                return LegoLinkFusionEligibility(False, "kv_head_layout_mismatch")
            if key.dtype != key_buffer.dtype or value.dtype != key_buffer.dtype:
                return LegoLinkFusionEligibility(False, "kv_dtype_mismatch")
    if key_buffer.dtype not in (torch.float16, torch.bfloat16):
        return LegoLinkFusionEligibility(False, "fp16_or_bf16_required")
    if not all(
        buffer.is_contiguous()
        for buffer in (*key_buffers, *value_buffers, *source_key_buffers, *source_value_buffers)
    ):
        return LegoLinkFusionEligibility(False, "contiguous_kv_buffers_required")
    key_head_dim = int(key_buffer.shape[-1])
    value_head_dim = int(value_buffer.shape[-1])
    if key_head_dim <= 0 or value_head_dim <= 0 or key_head_dim > 256 or value_head_dim > 256:
        return LegoLinkFusionEligibility(False, "head_dimension_out_of_range")
    token_count = int(source_slots.numel())
    if token_count == 0:
        return LegoLinkFusionEligibility(False, "empty_link")
    if any(
        int(tensor.numel()) != token_count
        for tensor in (destination_slots, local_positions, global_positions)
    ):
        return LegoLinkFusionEligibility(False, "token_map_length_mismatch")
    if repair_mask is not None:
        if not repair_mask.is_cuda:
            return LegoLinkFusionEligibility(False, "cuda_repair_mask_required")
        if int(repair_mask.numel()) != token_count:
            return LegoLinkFusionEligibility(False, "repair_mask_length_mismatch")
        if repair_mask.dtype not in (torch.bool, torch.uint8):
            return LegoLinkFusionEligibility(False, "boolean_repair_mask_required")
        if not repair_mask.is_contiguous():
            return LegoLinkFusionEligibility(False, "contiguous_repair_mask_required")
    if any(
        tensor.dtype not in (torch.int32, torch.int64)
        for tensor in (source_slots, destination_slots, local_positions, global_positions)
    ):
        return LegoLinkFusionEligibility(False, "integer_token_maps_required")
    rotary_dim = int(rotary_dim)
    if rotary_dim <= 0 or rotary_dim % 2:
        return LegoLinkFusionEligibility(False, "even_rotary_dim_required")
    if rotary_dim > key_head_dim:
        return LegoLinkFusionEligibility(False, "rotary_dim_exceeds_head_dim")
    if cos_sin_cache.ndim != 2 or int(cos_sin_cache.shape[1]) < rotary_dim:
        return LegoLinkFusionEligibility(False, "unsupported_cos_sin_cache")
    if cos_sin_cache.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return LegoLinkFusionEligibility(False, "unsupported_cos_sin_dtype")
    # The kernels read the token maps as dense arrays on the pool's device.
    device = key_buffer.device
    if any(
        tensor.device != device
        for tensor in (*tensors, *(() if repair_mask is None else (repair_mask,)))
    ):
        return LegoLinkFusionEligibility(False, "same_device_required")
    if not all(
        tensor.is_contiguous()
        for tensor in (source_slots, destination_slots, local_positions, global_positions)
    ):
        return LegoLinkFusionEligibility(False, "contiguous_token_maps_required")
    return LegoLinkFusionEligibility(True, "supported")


def check_fused_kv_link_eligibility(
    *,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    rotary_dim: int,
    repair_mask: torch.Tensor | None = None,
) -> LegoLinkFusionEligibility:
    """Can the HIP link run on these tensors? (legolink_triton.py:159-247)."""

    return _eligibility(
        [key_buffer],
        [value_buffer],
        source_slots,
        destination_slots,
        local_positions,
        global_positions,
        cos_sin_cache,
        rotary_dim,
        repair_mask,
    )


def _validate_index_ranges(
    num_slots: int,
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cache_rows: int,
    prefix_token_count: int,
    source_num_slots: int | None = None,
) -> None:
    """Optional host check (synchronises): the kernels skip out-of-range rows."""

    for name, tensor, limit in (
        ("source_slots", source_slots, num_slots if source_num_slots is None else source_num_slots),
        ("destination_slots", destination_slots, num_slots),
        ("local_positions", local_positions[prefix_token_count:], cache_rows),
        ("global_positions", global_positions[prefix_token_count:], cache_rows),
    ):
        if tensor.numel() and (int(tensor.min()) < 0 or int(tensor.max()) >= limit):
            raise IndexError(f"{name} has values outside [0, {limit})")


def _link_args(
    key_buffers: Sequence[torch.Tensor],
    value_buffers: Sequence[torch.Tensor],
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    prefix_token_count: int,
    rotary_dim: int,
    is_neox_style: bool,
    repair_mask: torch.Tensor | None,
    waves_per_block: int,
    layers_per_wave: int,
    kernel: int,
    layer_groups_per_block: int = 0,
    source_key_buffers: Sequence[torch.Tensor] = (),
    source_value_buffers: Sequence[torch.Tensor] = (),
    rounding: str = "fused",
    delta_staging: str = "auto",
) -> tuple[_native.LinkArgs, tuple[Any, ...]]:
    key_table = _native.pointer_table([buffer.data_ptr() for buffer in key_buffers])
    value_table = _native.pointer_table([buffer.data_ptr() for buffer in value_buffers])
    source_tables: tuple[Any, ...] = ()
    if source_key_buffers:
        source_tables = (
            _native.pointer_table([buffer.data_ptr() for buffer in source_key_buffers]),
            _native.pointer_table([buffer.data_ptr() for buffer in source_value_buffers]),
        )
    key_buffer, value_buffer = key_buffers[0], value_buffers[0]
    args = _native.LinkArgs()
    args.num_layers = len(key_buffers)
    args.key_layers = ctypes_address(key_table)
    args.value_layers = ctypes_address(value_table)
    args.num_slots = int(key_buffer.shape[0])
    args.num_heads = int(key_buffer.shape[1])
    args.key_head_dim = int(key_buffer.shape[2])
    args.value_head_dim = int(value_buffer.shape[2])
    args.kv_dtype = _KV_DTYPES[key_buffer.dtype]
    args.num_tokens = int(source_slots.numel())
    args.source_slots = source_slots.data_ptr()
    args.source_slots_dtype = _INDEX_DTYPES[source_slots.dtype]
    args.destination_slots = destination_slots.data_ptr()
    args.destination_slots_dtype = _INDEX_DTYPES[destination_slots.dtype]
    args.local_positions = local_positions.data_ptr()
    args.local_positions_dtype = _INDEX_DTYPES[local_positions.dtype]
    args.global_positions = global_positions.data_ptr()
    args.global_positions_dtype = _INDEX_DTYPES[global_positions.dtype]
    args.repair_mask = None if repair_mask is None else repair_mask.data_ptr()
    args.repair_mask_dtype = _native.DTYPE_UINT8
    args.cos_sin_cache = cos_sin_cache.data_ptr()
    args.cos_sin_dtype = _CACHE_DTYPES[cos_sin_cache.dtype]
    args.cos_sin_rows = int(cos_sin_cache.shape[0])
    args.cos_sin_cols = int(cos_sin_cache.shape[1])
    args.cos_sin_stride_row = int(cos_sin_cache.stride(0))
    args.cos_sin_stride_col = int(cos_sin_cache.stride(1))
    args.rotary_dim = int(rotary_dim)
    args.is_neox_style = 1 if is_neox_style else 0
    args.prefix_token_count = int(prefix_token_count)
    args.kernel = int(kernel)
    args.waves_per_block = int(waves_per_block)
    args.layers_per_wave = int(layers_per_wave)
    args.layer_groups_per_block = int(layer_groups_per_block)
    args.rounding = _rounding_code(rounding)
    if delta_staging not in DELTA_STAGINGS:
        raise ValueError(f"delta_staging must be one of {sorted(DELTA_STAGINGS)}, got {delta_staging!r}")
    args.delta_staging = DELTA_STAGINGS[delta_staging]
    if delta_staging == "workgroup":
        args.waves_per_block = 0  # the workgroup holds every layer group: the library sizes it
    if source_tables:
        args.source_key_layers = ctypes_address(source_tables[0])
        args.source_value_layers = ctypes_address(source_tables[1])
        args.source_num_slots = int(source_key_buffers[0].shape[0])
    # The pointer tables must outlive the call.
    return args, (key_table, value_table, *source_tables)


def ctypes_address(array: Any) -> int:
    return ctypes.addressof(array)


def _raise_unavailable(reason: str) -> None:
    raise RuntimeError(f"HIP LegoLink fusion is unavailable: {reason}")


class PreparedKVLink:
    """A validated link: the argument block is built once and every call
    enqueues the kernel with one C call (a few microseconds of host time).

    Arguments are those of ``fused_kv_link_layers_inplace``; the tensors are
    referenced, not copied, so their contents may change between calls (the
    kernel reads them when it runs) but their storage must stay alive and in
    place.

    ``rounding`` picks the rounding points of re-rotated K: "fused" (the
    reference's fused operator) or "eager" (its torch path); V and copied K are
    bit copies either way.

    ``delta_workspace`` (a device tensor of at least
    ``delta_workspace_bytes(tokens, rotary_dim)`` bytes) lets the library
    compute every token's delta once into a table and walk the rows layer by
    layer (``delta_staging="table"``); links that share one must not overlap.

    ``skipped_rows`` (a one-element int64 device tensor) receives, per call,
    the count of unmasked tokens the kernel skipped because a slot or position
    is out of range; the caller zeroes it and reads it after the stream's work.
    """

    def __init__(
        self,
        *,
        key_buffers: Sequence[torch.Tensor],
        value_buffers: Sequence[torch.Tensor],
        source_slots: torch.Tensor,
        destination_slots: torch.Tensor,
        local_positions: torch.Tensor,
        global_positions: torch.Tensor,
        cos_sin_cache: torch.Tensor,
        prefix_token_count: int,
        rotary_dim: int,
        is_neox_style: bool,
        repair_mask: torch.Tensor | None = None,
        block_size: int | None = None,
        num_warps: int | None = None,
        num_stages: int | None = None,
        layers_per_wave: int = 0,
        kernel: int = _native.KERNEL_AUTO,
        validate_indices: bool = False,
        layer_groups_per_block: int = 0,
        source_key_buffers: Sequence[torch.Tensor] | None = None,
        source_value_buffers: Sequence[torch.Tensor] | None = None,
        stream_source_rows: bool = False,
        rounding: str = "fused",
        delta_staging: str = "auto",
        skipped_rows: torch.Tensor | None = None,
        delta_workspace: torch.Tensor | None = None,
    ) -> None:
        key_buffers = list(key_buffers)
        value_buffers = list(value_buffers)
        source_key_buffers = list(source_key_buffers or ())
        source_value_buffers = list(source_value_buffers or ())
        if not key_buffers or len(key_buffers) != len(value_buffers):
            raise ValueError("key_buffers and value_buffers must be equal-length, non-empty")
        eligibility = _eligibility(
            key_buffers,
            value_buffers,
            source_slots,
            destination_slots,
            local_positions,
            global_positions,
            cos_sin_cache,
            rotary_dim,
            repair_mask,
            source_key_buffers,
            source_value_buffers,
        )
        if not eligibility.supported:
            _raise_unavailable(eligibility.reason)
        if not 0 <= int(prefix_token_count) <= int(source_slots.numel()):
            raise ValueError("prefix_token_count is outside the linked token range")
        key_buffer, value_buffer = key_buffers[0], value_buffers[0]
        work_items = int(key_buffer.shape[1]) * (
            int(rotary_dim) // 2
            + int(key_buffer.shape[2])
            - int(rotary_dim)
            + int(value_buffer.shape[2])
        )
        self.launch_config = resolve_fused_kv_launch_config(
            work_items=work_items,
            device=key_buffer.device,
            block_size=block_size,
            num_warps=num_warps,
            num_stages=num_stages,
        )
        if validate_indices:
            _validate_index_ranges(
                int(key_buffer.shape[0]),
                source_slots,
                destination_slots,
                local_positions,
                global_positions,
                int(cos_sin_cache.shape[0]),
                int(prefix_token_count),
                int(source_key_buffers[0].shape[0]) if source_key_buffers else None,
            )
        if repair_mask is not None and repair_mask.dtype == torch.bool:
            repair_mask = repair_mask.view(torch.uint8)
        self._args, self._tables = _link_args(
            key_buffers,
            value_buffers,
            source_slots,
            destination_slots,
            local_positions,
            global_positions,
            cos_sin_cache,
            prefix_token_count,
            rotary_dim,
            is_neox_style,
            repair_mask,
            self.launch_config.num_warps,
            layers_per_wave,
            kernel,
            layer_groups_per_block,
            source_key_buffers,
            source_value_buffers,
            rounding,
            delta_staging,
        )
        self.rounding = rounding
        if skipped_rows is not None:
            if (skipped_rows.dtype != torch.int64 or skipped_rows.numel() != 1
                    or skipped_rows.device != key_buffer.device):
                raise ValueError("skipped_rows must be a one-element int64 tensor on the link's device")
            self._args.skipped_rows = skipped_rows.data_ptr()
        if delta_workspace is not None:
            if not delta_workspace.is_contiguous() or delta_workspace.device != key_buffer.device:
                raise ValueError("delta_workspace must be a contiguous tensor on the link's device")
            self._args.delta_workspace = delta_workspace.data_ptr()
            self._args.delta_workspace_bytes = delta_workspace.numel() * delta_workspace.element_size()
        self._args.struct_size = ctypes.sizeof(_native.LinkArgs)
        # Rows read once (no source repeats within the launch) take non-temporal loads.
        self._args.stream_source_rows = 1 if stream_source_rows else 0
        # Keep every tensor the argument block points at alive.
        self._tensors = (
            key_buffers, value_buffers, source_slots, destination_slots,
            local_positions, global_positions, cos_sin_cache, repair_mask,
            source_key_buffers, source_value_buffers, skipped_rows, delta_workspace,
        )
        self.device = key_buffer.device
        try:
            info = _native.kv_link_describe(self._args)
        except _native.NativeCallError as error:
            self._raise_for(error)
        self.launch = _launch_record(info)
        self._lib = _native.load_library()
        self._args_ref = ctypes.byref(self._args)

    @staticmethod
    def _raise_for(error: _native.NativeCallError) -> None:
        if error.status == _native.LL_ERR_PREFIX_OUT_OF_RANGE:
            raise ValueError("prefix_token_count is outside the linked token range") from error
        if error.status in (_native.LL_ERR_LAUNCH_CONFIG, _native.LL_ERR_UNSUPPORTED_KERNEL):
            raise ValueError(str(error)) from error
        if error.status == _native.LL_ERR_HIP:
            raise RuntimeError(f"HIP LegoLink link launch failed: {error.detail}") from error
        _raise_unavailable(error.reason)

    def __call__(self, stream: torch.cuda.Stream | None = None) -> None:
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        status = self._lib.ll_kv_link(self._args_ref, ctypes.c_void_p(stream.cuda_stream))
        if status != _native.LL_OK:
            self._raise_for(
                _native.NativeCallError(
                    status,
                    self._lib.ll_status_reason(status).decode(),
                    self._lib.ll_last_error().decode(),
                )
            )


def fused_kv_link_layers_inplace(
    *,
    key_buffers: Sequence[torch.Tensor],
    value_buffers: Sequence[torch.Tensor],
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    prefix_token_count: int,
    rotary_dim: int,
    is_neox_style: bool,
    repair_mask: torch.Tensor | None = None,
    block_size: int | None = None,
    num_warps: int | None = None,
    num_stages: int | None = None,
    layers_per_wave: int = 0,
    kernel: int = _native.KERNEL_AUTO,
    validate_indices: bool = False,
    layer_groups_per_block: int = 0,
    source_key_buffers: Sequence[torch.Tensor] | None = None,
    source_value_buffers: Sequence[torch.Tensor] | None = None,
    stream_source_rows: bool = False,
    rounding: str = "fused",
    delta_staging: str = "auto",
    skipped_rows: torch.Tensor | None = None,
    delta_workspace: torch.Tensor | None = None,
) -> None:
    """Link every layer in ``key_buffers``/``value_buffers`` with one launch per
    64 layers, on the current stream.  Per layer the result equals
    ``fused_kv_link_inplace``.  With ``source_key_buffers``/``source_value_buffers``
    (one per layer, same row layout) the source rows are read from that pool
    instead of the destination pool.  ``stream_source_rows`` says that no source
    row repeats within the link (non-temporal loads; the result is the same).
    ``rounding="eager"`` gives the reference's torch-path result instead
    (``_remap_key_positions``, pic_runtime.py:6025-6058)."""

    prepared = PreparedKVLink(
        key_buffers=key_buffers,
        value_buffers=value_buffers,
        source_slots=source_slots,
        destination_slots=destination_slots,
        local_positions=local_positions,
        global_positions=global_positions,
        cos_sin_cache=cos_sin_cache,
        prefix_token_count=prefix_token_count,
        rotary_dim=rotary_dim,
        is_neox_style=is_neox_style,
        repair_mask=repair_mask,
        block_size=block_size,
        num_warps=num_warps,
        num_stages=num_stages,
        layers_per_wave=layers_per_wave,
        kernel=kernel,
        validate_indices=validate_indices,
        layer_groups_per_block=layer_groups_per_block,
        source_key_buffers=source_key_buffers,
        source_value_buffers=source_value_buffers,
        stream_source_rows=stream_source_rows,
        rounding=rounding,
        delta_staging=delta_staging,
        skipped_rows=skipped_rows,
        delta_workspace=delta_workspace,
    )
    prepared()


def fused_kv_link_inplace(
    *,
    key_buffer: torch.Tensor,
    value_buffer: torch.Tensor,
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    prefix_token_count: int,
    rotary_dim: int,
    is_neox_style: bool,
    repair_mask: torch.Tensor | None = None,
    block_size: int | None = None,
    num_warps: int | None = None,
    num_stages: int | None = None,
) -> None:
    """Link one layer in place (legolink_triton.py:550-645).

    For every linked token t (skipped when ``repair_mask[t]`` is set):
    V[dst[t]] = V[src[t]]; K[dst[t]] = K[src[t]] for t < prefix_token_count,
    otherwise K[src[t]] re-rotated from ``local_positions[t]`` to
    ``global_positions[t]``.  Raises RuntimeError with the eligibility reason
    and ValueError for a bad prefix or launch configuration, like the reference.
    """

    fused_kv_link_layers_inplace(
        key_buffers=[key_buffer],
        value_buffers=[value_buffer],
        source_slots=source_slots,
        destination_slots=destination_slots,
        local_positions=local_positions,
        global_positions=global_positions,
        cos_sin_cache=cos_sin_cache,
        prefix_token_count=prefix_token_count,
        rotary_dim=rotary_dim,
        is_neox_style=is_neox_style,
        repair_mask=repair_mask,
        block_size=block_size,
        num_warps=num_warps,
        num_stages=num_stages,
    )


def describe_link_launch(
    *,
    key_buffers: Sequence[torch.Tensor],
    value_buffers: Sequence[torch.Tensor],
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    prefix_token_count: int,
    rotary_dim: int,
    is_neox_style: bool,
    repair_mask: torch.Tensor | None = None,
    num_warps: int = 4,
    layers_per_wave: int = 0,
    kernel: int = _native.KERNEL_AUTO,
    layer_groups_per_block: int = 0,
    rounding: str = "fused",
    delta_staging: str = "auto",
    stream_source_rows: bool = False,
    delta_workspace: torch.Tensor | None = None,
) -> dict[str, Any]:
    """Kernel and launch shape the link would use (no GPU work, no device needed)."""

    if repair_mask is not None and repair_mask.dtype == torch.bool:
        repair_mask = repair_mask.view(torch.uint8)
    args, keepalive = _link_args(
        list(key_buffers),
        list(value_buffers),
        source_slots,
        destination_slots,
        local_positions,
        global_positions,
        cos_sin_cache,
        prefix_token_count,
        rotary_dim,
        is_neox_style,
        repair_mask,
        num_warps,
        layers_per_wave,
        kernel,
        layer_groups_per_block,
        rounding=rounding,
        delta_staging=delta_staging,
    )
    args.stream_source_rows = 1 if stream_source_rows else 0
    if delta_workspace is not None:
        args.delta_workspace = delta_workspace.data_ptr()
        args.delta_workspace_bytes = delta_workspace.numel() * delta_workspace.element_size()
    info = _native.kv_link_describe(args)
    del keepalive
    return _launch_record(info)


class PreparedKVScatter:
    """A validated repaired-row write-back; each call enqueues one kernel launch
    per 64 layers.

    ``repaired_keys`` is [num_layers, rows, heads, key_head_dim] (or
    [rows, heads, key_head_dim] for a single layer) with dense rows; the layer
    stride may be anything.  Semantics of write_repaired_kv
    (tests/pic/reference/repair_reference.py:14-25) applied to every layer:
    K_l[destination_slots[r]] = repaired_keys[l, r], V likewise.
    """

    def __init__(
        self,
        *,
        key_buffers: Sequence[torch.Tensor],
        value_buffers: Sequence[torch.Tensor],
        destination_slots: torch.Tensor,
        repaired_keys: torch.Tensor,
        repaired_values: torch.Tensor,
        num_warps: int = 4,
    ) -> None:
        key_buffers = list(key_buffers)
        value_buffers = list(value_buffers)
        if not key_buffers or len(key_buffers) != len(value_buffers):
            raise ValueError("key_buffers and value_buffers must be equal-length, non-empty")
        if repaired_keys.ndim == 3:
            repaired_keys = repaired_keys.unsqueeze(0)
        if repaired_values.ndim == 3:
            repaired_values = repaired_values.unsqueeze(0)
        key_buffer, value_buffer = key_buffers[0], value_buffers[0]
        layers = len(key_buffers)
        rows = int(destination_slots.numel())
        if not _native.library_available():
            _raise_unavailable(NATIVE_UNAVAILABLE_REASON)
        tensors = (*key_buffers, *value_buffers, destination_slots, repaired_keys, repaired_values)
        if not all(tensor.is_cuda and tensor.device == key_buffer.device for tensor in tensors):
            _raise_unavailable("cuda_tensors_required")
        for key, value in zip(key_buffers, value_buffers, strict=True):
            if key.ndim != 3 or value.ndim != 3:
                _raise_unavailable("mha_3d_kv_buffers_required")
            if key.shape != key_buffer.shape or value.shape != value_buffer.shape or (
                key.shape[:2] != value.shape[:2]
            ):
                _raise_unavailable("kv_head_layout_mismatch")
            if key.dtype != key_buffer.dtype or value.dtype != key_buffer.dtype:
                _raise_unavailable("kv_dtype_mismatch")
            if not key.is_contiguous() or not value.is_contiguous():
                _raise_unavailable("contiguous_kv_buffers_required")
        if key_buffer.dtype not in _KV_DTYPES:
            _raise_unavailable("fp16_or_bf16_required")
        if destination_slots.dtype not in _INDEX_DTYPES or not destination_slots.is_contiguous():
            _raise_unavailable("integer_token_maps_required")
        expected_k = (layers, rows, int(key_buffer.shape[1]), int(key_buffer.shape[2]))
        expected_v = (layers, rows, int(value_buffer.shape[1]), int(value_buffer.shape[2]))
        if tuple(repaired_keys.shape) != expected_k or tuple(repaired_values.shape) != expected_v:
            raise ValueError(
                f"repaired rows must be {expected_k} / {expected_v}, got "
                f"{tuple(repaired_keys.shape)} / {tuple(repaired_values.shape)}"
            )
        if repaired_keys.dtype != key_buffer.dtype or repaired_values.dtype != key_buffer.dtype:
            _raise_unavailable("kv_dtype_mismatch")
        if not repaired_keys[0].is_contiguous() or not repaired_values[0].is_contiguous():
            raise ValueError("repaired rows of each layer must be dense")
        self.rows = rows
        self.device = key_buffer.device
        self._tables = (
            _native.pointer_table([buffer.data_ptr() for buffer in key_buffers]),
            _native.pointer_table([buffer.data_ptr() for buffer in value_buffers]),
        )
        args = _native.ScatterArgs()
        args.struct_size = ctypes.sizeof(_native.ScatterArgs)
        args.num_layers = layers
        args.key_layers = ctypes_address(self._tables[0])
        args.value_layers = ctypes_address(self._tables[1])
        args.num_slots = int(key_buffer.shape[0])
        args.num_heads = int(key_buffer.shape[1])
        args.key_head_dim = int(key_buffer.shape[2])
        args.value_head_dim = int(value_buffer.shape[2])
        args.kv_dtype = _KV_DTYPES[key_buffer.dtype]
        args.num_rows = rows
        args.destination_slots = destination_slots.data_ptr()
        args.destination_slots_dtype = _INDEX_DTYPES[destination_slots.dtype]
        args.repaired_key = repaired_keys.data_ptr()
        args.repaired_key_layer_stride = int(repaired_keys.stride(0)) if layers > 1 else 0
        args.repaired_value = repaired_values.data_ptr()
        args.repaired_value_layer_stride = int(repaired_values.stride(0)) if layers > 1 else 0
        args.waves_per_block = int(num_warps)
        self._args = args
        self._args_ref = ctypes.byref(args)
        self._tensors = tensors
        self._lib = _native.load_library()

    def __call__(self, stream: torch.cuda.Stream | None = None) -> None:
        if self.rows == 0:
            return
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        status = self._lib.ll_kv_scatter_rows(self._args_ref, ctypes.c_void_p(stream.cuda_stream))
        if status != _native.LL_OK:
            reason = self._lib.ll_status_reason(status).decode()
            detail = self._lib.ll_last_error().decode()
            if status == _native.LL_ERR_HIP:
                raise RuntimeError(f"HIP LegoLink scatter launch failed: {detail}")
            _raise_unavailable(reason)


def scatter_kv_rows_inplace(
    *,
    key_buffers: Sequence[torch.Tensor],
    value_buffers: Sequence[torch.Tensor],
    destination_slots: torch.Tensor,
    repaired_keys: torch.Tensor,
    repaired_values: torch.Tensor,
    num_warps: int = 4,
) -> None:
    """Write repaired rows on the current stream: K_l[destination_slots[r]] =
    repaired_keys[l, r] (and V).  See ``PreparedKVScatter``."""

    PreparedKVScatter(
        key_buffers=key_buffers,
        value_buffers=value_buffers,
        destination_slots=destination_slots,
        repaired_keys=repaired_keys,
        repaired_values=repaired_values,
        num_warps=num_warps,
    )()
