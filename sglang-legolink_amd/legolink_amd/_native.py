"""ctypes binding of ``liblegolink_kv.so`` (the C ABI in ``include/legolink_kv.h``).

The library is built in-tree for gfx950 (``legolink_amd.build``).  It links
against ``libamdhip64.so.7``; torch is imported before the library is opened so
that the dynamic loader binds those symbols to the HIP runtime torch already
loaded, and device pointers and streams handed over from torch are valid in
the library.

There is no fallback: when the library is missing every entry raises
``NativeLibraryUnavailable``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
# LEGOLINK_KV_LIBRARY names another build of the library (the host-sanitized
# one of the CPU sanitizer test).
LIB_PATH = Path(os.environ.get("LEGOLINK_KV_LIBRARY") or LIB_DIR / "liblegolink_kv.so")
ABI_VERSION = 17

# Element type codes (include/legolink_kv.h).
DTYPE_FLOAT16 = 1
DTYPE_BFLOAT16 = 2
DTYPE_FLOAT32 = 3
DTYPE_INT32 = 4
DTYPE_INT64 = 5
DTYPE_UINT8 = 6

ROUNDING_FUSED = 0
ROUNDING_EAGER = 1

DELTA_AUTO = 0
DELTA_PER_WAVE = 1
DELTA_WORKGROUP = 2
DELTA_TABLE = 3

KERNEL_AUTO = 0
KERNEL_VECTOR = 1
KERNEL_GENERIC = 2

# Status codes.
LL_OK = 0
LL_ERR_INVALID_ARGUMENT = -1
LL_ERR_PREFIX_OUT_OF_RANGE = -17
LL_ERR_LAUNCH_CONFIG = -18
LL_ERR_UNSUPPORTED_KERNEL = -19
LL_ERR_HIP = -20

EXPORTED_SYMBOLS = (
    "ll_kv_link",
    "ll_kv_link_describe",
    "ll_kv_scatter_rows",
    "ll_status_reason",
    "ll_last_error",
    "ll_abi_version",
    "ll_kv_link_args_size",
    "ll_kv_scatter_args_size",
    "ll_kv_build_link_maps",
    "ll_link_maps_args_size",
    "ll_order_link_maps",
    "ll_order_maps_args_size",
    "ll_repair_attention_plan",
    "ll_repair_attention",
    "ll_repair_attention_args_size",
    "ll_repair_attention_noalloc",
    "ll_repair_scratch_bytes",
    "ll_plan_link_runs",
)

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


class LinkArgs(ctypes.Structure):
    """Mirror of ``ll_kv_link_args``."""

    _fields_ = [
        ("struct_size", _i64),
        ("num_layers", _i64),
        ("key_layers", _ptr),
        ("value_layers", _ptr),
        ("num_slots", _i64),
        ("num_heads", _i64),
        ("key_head_dim", _i64),
        ("value_head_dim", _i64),
        ("kv_dtype", _i64),
        ("num_tokens", _i64),
        ("source_slots", _ptr),
        ("source_slots_dtype", _i64),
        ("destination_slots", _ptr),
        ("destination_slots_dtype", _i64),
        ("local_positions", _ptr),
        ("local_positions_dtype", _i64),
        ("global_positions", _ptr),
        ("global_positions_dtype", _i64),
        ("repair_mask", _ptr),
        ("repair_mask_dtype", _i64),
        ("cos_sin_cache", _ptr),
        ("cos_sin_dtype", _i64),
        ("cos_sin_rows", _i64),
        ("cos_sin_cols", _i64),
        ("cos_sin_stride_row", _i64),
        ("cos_sin_stride_col", _i64),
        ("rotary_dim", _i64),
        ("is_neox_style", _i64),
        ("prefix_token_count", _i64),
        ("kernel", _i64),
        ("waves_per_block", _i64),
        ("layers_per_wave", _i64),
        ("layer_groups_per_block", _i64),
        ("source_key_layers", _ptr),
        ("source_value_layers", _ptr),
        ("source_num_slots", _i64),
        ("stream_source_rows", _i64),
        ("rounding", _i64),
        ("delta_staging", _i64),
        ("skipped_rows", _ptr),
        ("delta_workspace", _ptr),
        ("delta_workspace_bytes", _i64),
    ]


class ScatterArgs(ctypes.Structure):
    """Mirror of ``ll_kv_scatter_args``."""

    _fields_ = [
        ("struct_size", _i64),
        ("num_layers", _i64),
        ("key_layers", _ptr),
        ("value_layers", _ptr),
        ("num_slots", _i64),
        ("num_heads", _i64),
        ("key_head_dim", _i64),
        ("value_head_dim", _i64),
        ("kv_dtype", _i64),
        ("num_rows", _i64),
        ("destination_slots", _ptr),
        ("destination_slots_dtype", _i64),
        ("repaired_key", _ptr),
        ("repaired_key_layer_stride", _i64),
        ("repaired_value", _ptr),
        ("repaired_value_layer_stride", _i64),
        ("waves_per_block", _i64),
    ]


class LinkSegment(ctypes.Structure):
    """Mirror of ``ll_link_segment`` (eleven 8-byte fields: an int64 ``[n, 11]``
    array has the same memory layout as ``n`` of these)."""

    _fields_ = [
        ("source_slots", _ptr),
        ("local_positions", _ptr),
        ("token_count", _i64),
        ("start_token", _i64),
        ("destination_start", _i64),
        ("local_start", _i64),
        ("repair_begin", _i64),
        ("repair_end", _i64),
        ("map_set", _i64),
        ("map_offset", _i64),
        ("repair_offset", _i64),
    ]


SEGMENT_FIELDS = tuple(name for name, _ in LinkSegment._fields_)


class LinkBlock(ctypes.Structure):
    """Mirror of ``ll_link_block`` (eight 8-byte fields: an int64 ``[n, 8]``
    array has the same memory layout as ``n`` of these)."""

    _fields_ = [
        ("source_slots", _ptr),
        ("local_positions", _ptr),
        ("token_count", _i64),
        ("start_token", _i64),
        ("destination_base", _i64),
        ("local_start", _i64),
        ("map_set", _i64),
        ("leading", _i64),
    ]


BLOCK_FIELDS = tuple(name for name, _ in LinkBlock._fields_)


class LinkRunPlanInfo(ctypes.Structure):
    """Mirror of ``ll_link_run_plan_info``."""

    _fields_ = [
        ("num_segments", _i64),
        ("map_count", _i64 * 2),
        ("set_repair_rows", _i64 * 2),
        ("set_prefix", _i64 * 2),
        ("repair_count", _i64),
    ]


class LinkMapsArgs(ctypes.Structure):
    """Mirror of ``ll_link_maps_args``."""

    _fields_ = [
        ("struct_size", _i64),
        ("num_segments", _i64),
        ("segments", _ptr),
        ("destination_slots", _ptr),
        ("destination_slots_dtype", _i64),
        ("num_destination_slots", _i64),
        ("maps", _ptr * 2),
        ("map_capacity", _i64 * 2),
        ("repair_mask", _ptr * 2),
        ("repair_destination_slots", _ptr),
        ("repair_capacity", _i64),
        ("device_segments", _ptr),
    ]


# Visit order of a map set (ll_order_link_maps).
ORDER_BUCKETS = 16384
ORDER_WORKSPACE_BYTES = 8 * ORDER_BUCKETS + 256


class OrderMapsArgs(ctypes.Structure):
    """Mirror of ``ll_order_maps_args``."""

    _fields_ = [
        ("struct_size", _i64),
        ("maps", _ptr),
        ("mask", _ptr),
        ("capacity", _i64),
        ("count", _i64),
        ("prefix", _i64),
        ("num_slots", _i64),
        ("out_maps", _ptr),
        ("out_mask", _ptr),
        ("workspace", _ptr),
        ("workspace_bytes", _i64),
        ("key_row", _i64),
    ]


class RepairRow(ctypes.Structure):
    """Mirror of ``ll_repair_row`` (four int64: an int64 ``[n, 4]`` array has the
    same memory layout as ``n`` of these)."""

    _fields_ = [
        ("query_index", _i64),
        ("query_start", _i64),
        ("query_count", _i64),
        ("kv_offset", _i64),
    ]


class RepairPlanInfo(ctypes.Structure):
    """Mirror of ``ll_repair_attention_plan_info``."""

    _fields_ = [
        ("num_items", _i64),
        ("num_combine", _i64),
        ("workspace_items", _i64),
        ("split_tokens", _i64),
        ("num_queries", _i64),
    ]


class RepairAttentionArgs(ctypes.Structure):
    """Mirror of ``ll_repair_attention_args``."""

    _fields_ = [
        ("struct_size", _i64),
        ("query", _ptr),
        ("output", _ptr),
        ("num_queries", _i64),
        ("key_buffer", _ptr),
        ("value_buffer", _ptr),
        ("num_slots", _i64),
        ("num_q_heads", _i64),
        ("num_kv_heads", _i64),
        ("head_dim", _i64),
        ("kv_dtype", _i64),
        ("softmax_scale", ctypes.c_double),
        ("kv_slots", _ptr),
        ("kv_slots_dtype", _i64),
        ("kv_slots_len", _i64),
        ("items", _ptr),
        ("num_items", _i64),
        ("combine", _ptr),
        ("num_combine", _i64),
        ("query_positions", _ptr),
        ("workspace", _ptr),
        ("workspace_items", _i64),
    ]


REPAIR_ITEM_INTS = 86
REPAIR_ITEM_HEADER = 6  # kv_offset, kv_begin, kv_end, tiles, first pair's head, pair count
REPAIR_TILE_INTS = 5   # per tile of an item: first query, lowest position, count, partial, key end
REPAIR_COMBINE_INTS = 4


class LaunchInfo(ctypes.Structure):
    """Mirror of ``ll_launch_info``."""

    _fields_ = [
        ("kernel", _i64),
        ("launches", _i64),
        ("grid_x", _i64),
        ("grid_y", _i64),
        ("block_threads", _i64),
        ("layers_per_wave", _i64),
        ("layer_groups_per_block", _i64),
        ("delta_staging", _i64),
    ]


class NativeLibraryUnavailable(RuntimeError):
    """``liblegolink_kv.so`` is not built or cannot be loaded."""


class NativeCallError(RuntimeError):
    """A library entry returned a negative status."""

    def __init__(self, status: int, reason: str, message: str) -> None:
        super().__init__(f"{reason}: {message}" if message else reason)
        self.status = status
        self.reason = reason
        self.detail = message


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load_library() -> ctypes.CDLL:
    """Open the library once, verify its ABI, and return the handle."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (binds libamdhip64.so.7 to torch's copy first)

        if not LIB_PATH.is_file():
            raise NativeLibraryUnavailable(
                f"{LIB_PATH} is not built; build it with "
                "`python -m legolink_amd.build` (hipcc --offload-arch=gfx950)"
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as error:
            raise NativeLibraryUnavailable(f"cannot load {LIB_PATH}: {error}") from error
        lib.ll_kv_link.argtypes = [ctypes.POINTER(LinkArgs), _ptr]
        lib.ll_kv_link.restype = ctypes.c_int
        lib.ll_kv_link_describe.argtypes = [ctypes.POINTER(LinkArgs), ctypes.POINTER(LaunchInfo)]
        lib.ll_kv_link_describe.restype = ctypes.c_int
        lib.ll_kv_scatter_rows.argtypes = [ctypes.POINTER(ScatterArgs), _ptr]
        lib.ll_kv_scatter_rows.restype = ctypes.c_int
        lib.ll_status_reason.argtypes = [ctypes.c_int]
        lib.ll_status_reason.restype = ctypes.c_char_p
        lib.ll_last_error.argtypes = []
        lib.ll_last_error.restype = ctypes.c_char_p
        lib.ll_abi_version.argtypes = []
        lib.ll_abi_version.restype = ctypes.c_int
        lib.ll_kv_link_args_size.argtypes = []
        lib.ll_kv_link_args_size.restype = _i64
        lib.ll_kv_scatter_args_size.argtypes = []
        lib.ll_kv_scatter_args_size.restype = _i64
        lib.ll_kv_build_link_maps.argtypes = [ctypes.POINTER(LinkMapsArgs), _ptr]
        lib.ll_kv_build_link_maps.restype = ctypes.c_int
        lib.ll_link_maps_args_size.argtypes = []
        lib.ll_link_maps_args_size.restype = _i64
        lib.ll_order_link_maps.argtypes = [ctypes.POINTER(OrderMapsArgs), _ptr]
        lib.ll_order_link_maps.restype = ctypes.c_int
        lib.ll_order_maps_args_size.argtypes = []
        lib.ll_order_maps_args_size.restype = _i64
        lib.ll_repair_attention_plan.argtypes = [_ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64,
                                                 _ptr, _i64, ctypes.POINTER(RepairPlanInfo)]
        lib.ll_repair_attention_plan.restype = ctypes.c_int
        lib.ll_repair_attention.argtypes = [ctypes.POINTER(RepairAttentionArgs), _ptr]
        lib.ll_repair_attention.restype = ctypes.c_int
        lib.ll_repair_attention_args_size.argtypes = []
        lib.ll_repair_attention_args_size.restype = _i64
        lib.ll_plan_link_runs.argtypes = [_ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _i64,
                                          ctypes.POINTER(LinkRunPlanInfo)]
        lib.ll_plan_link_runs.restype = ctypes.c_int
        lib.ll_repair_attention_noalloc.argtypes = [ctypes.POINTER(RepairAttentionArgs), _ptr]
        lib.ll_repair_attention_noalloc.restype = ctypes.c_int
        lib.ll_repair_scratch_bytes.argtypes = []
        lib.ll_repair_scratch_bytes.restype = _i64
        if lib.ll_abi_version() != ABI_VERSION:
            raise NativeLibraryUnavailable(
                f"{LIB_PATH} has ABI {lib.ll_abi_version()}, expected {ABI_VERSION}; rebuild it"
            )
        if (lib.ll_kv_link_args_size() != ctypes.sizeof(LinkArgs)
                or lib.ll_kv_scatter_args_size() != ctypes.sizeof(ScatterArgs)
                or lib.ll_link_maps_args_size() != ctypes.sizeof(LinkMapsArgs)
                or lib.ll_order_maps_args_size() != ctypes.sizeof(OrderMapsArgs)
                or lib.ll_repair_attention_args_size() != ctypes.sizeof(RepairAttentionArgs)):
            raise NativeLibraryUnavailable(f"{LIB_PATH} struct layout differs; rebuild it")
        _lib = lib
        return lib


def library_available() -> bool:
    try:
        load_library()
    except NativeLibraryUnavailable:
        return False
    return True


def status_reason(status: int) -> str:
    return load_library().ll_status_reason(int(status)).decode()


def _check(status: int) -> None:
    if status != LL_OK:
        lib = load_library()
        raise NativeCallError(
            status, lib.ll_status_reason(status).decode(), lib.ll_last_error().decode()
        )


def pointer_table(pointers: list[int]) -> ctypes.Array:
    """Host array of device pointers for the per-layer tables."""

    table = (ctypes.c_void_p * len(pointers))()
    for index, value in enumerate(pointers):
        table[index] = int(value)
    return table


def kv_link(args: LinkArgs, stream: int) -> None:
    args.struct_size = ctypes.sizeof(LinkArgs)
    _check(load_library().ll_kv_link(ctypes.byref(args), _ptr(int(stream))))


def kv_link_describe(args: LinkArgs) -> LaunchInfo:
    args.struct_size = ctypes.sizeof(LinkArgs)
    info = LaunchInfo()
    _check(load_library().ll_kv_link_describe(ctypes.byref(args), ctypes.byref(info)))
    return info


def kv_build_link_maps(args: LinkMapsArgs, stream: int) -> None:
    args.struct_size = ctypes.sizeof(LinkMapsArgs)
    _check(load_library().ll_kv_build_link_maps(ctypes.byref(args), _ptr(int(stream))))


def order_link_maps(args: OrderMapsArgs, stream: int) -> None:
    args.struct_size = ctypes.sizeof(OrderMapsArgs)
    _check(load_library().ll_order_link_maps(ctypes.byref(args), _ptr(int(stream))))


def repair_attention_plan(rows, num_q_heads: int, num_kv_heads: int, split_tokens: int = 0):
    """Host planning: returns (items int32 [n, 86], combine int32 [m, 4],
    positions int32 [num_queries], info)."""

    import numpy as np

    rows = np.ascontiguousarray(np.asarray(rows, dtype=np.int64).reshape(-1, 4))
    lib = load_library()
    info = RepairPlanInfo()
    rows_ptr = rows.ctypes.data if rows.size else None
    _check(lib.ll_repair_attention_plan(rows_ptr, rows.shape[0], int(num_q_heads), int(num_kv_heads),
                                        int(split_tokens), None, 0, None, 0, None, 0, ctypes.byref(info)))
    items = np.empty((info.num_items, REPAIR_ITEM_INTS), dtype=np.int32)
    combine = np.empty((info.num_combine, REPAIR_COMBINE_INTS), dtype=np.int32)
    positions = np.empty(info.num_queries, dtype=np.int32)
    # The sizing call chose the chunk length: the filling call takes it as
    # given instead of searching again (same plan, half the host time).
    chosen = int(info.split_tokens)
    _check(lib.ll_repair_attention_plan(rows_ptr, rows.shape[0], int(num_q_heads), int(num_kv_heads),
                                        chosen, items.ctypes.data if items.size else None,
                                        info.num_items,
                                        combine.ctypes.data if combine.size else None, info.num_combine,
                                        positions.ctypes.data if positions.size else None, positions.size,
                                        ctypes.byref(info)))
    return items, combine, positions, info


def plan_link_runs(blocks, repair_positions, compact: bool):
    """ll_plan_link_runs over ``blocks`` (int64 ``[B, 8]`` ll_link_block
    records) and ``repair_positions`` (int64 ``[R]``): returns the runs (int64
    ``[S, 11]`` ll_link_segment records), the block of every run, the repair
    rows' concatenation offsets and the plan info."""

    import numpy as np

    blocks = np.ascontiguousarray(blocks, dtype=np.int64)
    repair_positions = np.ascontiguousarray(repair_positions, dtype=np.int64)
    capacity = blocks.shape[0] + repair_positions.size
    segments = np.empty((capacity, len(SEGMENT_FIELDS)), dtype=np.int64)
    segment_blocks = np.empty(capacity, dtype=np.int64)
    repair_offsets = np.empty(repair_positions.size, dtype=np.int64)
    info = LinkRunPlanInfo()
    _check(load_library().ll_plan_link_runs(
        blocks.ctypes.data if blocks.size else None, blocks.shape[0],
        repair_positions.ctypes.data if repair_positions.size else None, repair_positions.size,
        1 if compact else 0, segments.ctypes.data if capacity else None, capacity,
        segment_blocks.ctypes.data if capacity else None,
        repair_offsets.ctypes.data if repair_offsets.size else None, repair_offsets.size,
        ctypes.byref(info)))
    count = int(info.num_segments)
    return segments[:count], segment_blocks[:count], repair_offsets[: int(info.repair_count)], info


def repair_attention(args: RepairAttentionArgs, stream: int) -> None:
    args.struct_size = ctypes.sizeof(RepairAttentionArgs)
    _check(load_library().ll_repair_attention(ctypes.byref(args), _ptr(int(stream))))


def repair_attention_noalloc(args: RepairAttentionArgs, stream: int) -> None:
    """ll_repair_attention_noalloc: the split partials go to the library's
    device scratch array (``args.workspace`` must be NULL)."""

    args.struct_size = ctypes.sizeof(RepairAttentionArgs)
    _check(load_library().ll_repair_attention_noalloc(ctypes.byref(args), _ptr(int(stream))))


def repair_scratch_bytes() -> int:
    return int(load_library().ll_repair_scratch_bytes())
