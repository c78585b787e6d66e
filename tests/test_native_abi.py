"""The C-ABI library: it loads, exports every declared symbol, and validates
arguments before touching a device (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from legolink_amd import _native, kv_link
from legolink_amd.rope import build_cos_sin_cache

HEADER = Path(__file__).resolve().parents[1] / "include" / "legolink_kv.h"

# Reason strings of check_fused_kv_link_eligibility
# (patched_sglang_files/python/sglang/srt/legolink_triton.py:159-247).
REFERENCE_REASONS = {
    "mha_3d_kv_buffers_required", "kv_head_layout_mismatch", "kv_dtype_mismatch",
    "fp16_or_bf16_required", "contiguous_kv_buffers_required", "head_dimension_out_of_range",
    "empty_link", "token_map_length_mismatch", "repair_mask_length_mismatch",
    "boolean_repair_mask_required", "integer_token_maps_required", "even_rotary_dim_required",
    "rotary_dim_exceeds_head_dim", "unsupported_cos_sin_cache", "unsupported_cos_sin_dtype",
}


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(ll_\w+)\s*\(", text, re.MULTILINE)))


def test_library_loads_with_matching_abi():
    lib = _native.load_library()
    assert lib.ll_abi_version() == _native.ABI_VERSION
    assert lib.ll_kv_link_args_size() == ctypes.sizeof(_native.LinkArgs)
    assert lib.ll_kv_scatter_args_size() == ctypes.sizeof(_native.ScatterArgs)


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert set(names) == set(_native.EXPORTED_SYMBOLS), names
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    for name in names:
        assert hasattr(lib, name), name


def test_status_codes_map_to_reference_reasons():
    header = HEADER.read_text()
    codes = dict((name, int(value)) for name, value in re.findall(r"(LL_ERR_\w+)\s*=\s*(-\d+)", header))
    reasons = {name: _native.status_reason(code) for name, code in codes.items()}
    assert REFERENCE_REASONS <= set(reasons.values())
    assert len(set(reasons.values())) == len(reasons)  # one reason per code
    assert _native.status_reason(0) == "supported"


def _cpu_args(**overrides):
    keys = [torch.zeros(64, 4, 128, dtype=torch.bfloat16) for _ in range(2)]
    values = [torch.zeros(64, 4, 128, dtype=torch.bfloat16) for _ in range(2)]
    kwargs = dict(
        key_buffers=keys, value_buffers=values, source_slots=torch.arange(8),
        destination_slots=torch.arange(8, 16), local_positions=torch.arange(8),
        global_positions=torch.arange(8) + 3, cos_sin_cache=build_cos_sin_cache(32, 128),
        prefix_token_count=0, rotary_dim=128, is_neox_style=True, repair_mask=None,
        waves_per_block=4, layers_per_wave=0, kernel=0,
    )
    kwargs.update(overrides)
    ordered = [kwargs[name] for name in (
        "key_buffers", "value_buffers", "source_slots", "destination_slots", "local_positions",
        "global_positions", "cos_sin_cache", "prefix_token_count", "rotary_dim", "is_neox_style",
        "repair_mask", "waves_per_block", "layers_per_wave", "kernel")]
    return kv_link._link_args(*ordered)


@pytest.mark.parametrize("overrides,reason", [
    (dict(rotary_dim=7), "even_rotary_dim_required"),
    (dict(rotary_dim=130), "rotary_dim_exceeds_head_dim"),
    (dict(prefix_token_count=9), "prefix_token_count_out_of_range"),
    (dict(waves_per_block=3), "invalid_launch_config"),
    (dict(source_slots=torch.arange(0)), "empty_link"),
])
def test_invalid_arguments_are_rejected_before_any_launch(overrides, reason):
    args, keepalive = _cpu_args(**overrides)
    with pytest.raises(_native.NativeCallError) as error:
        _native.kv_link(args, 0)
    assert error.value.reason == reason
    del keepalive


def test_null_struct_and_bad_struct_size_are_rejected():
    lib = _native.load_library()
    assert lib.ll_kv_link(None, None) == _native.LL_ERR_INVALID_ARGUMENT
    args, keepalive = _cpu_args()
    args.struct_size = 8
    assert lib.ll_kv_link(ctypes.byref(args), None) == _native.LL_ERR_INVALID_ARGUMENT
    assert "struct_size" in lib.ll_last_error().decode()
    assert lib.ll_kv_scatter_rows(None, None) == _native.LL_ERR_INVALID_ARGUMENT
    del keepalive


def test_kernel_choice_and_launch_shape():
    # Qwen2.5-7B: 4 heads x 128 dims = 64 chunks of 16 bytes per row = one wave per token.
    args, keepalive = _cpu_args(source_slots=torch.arange(32768), destination_slots=torch.arange(32768),
                                local_positions=torch.arange(32768), global_positions=torch.arange(32768))
    args.delta_staging = _native.DELTA_PER_WAVE
    info = _native.kv_link_describe(args)
    assert info.kernel == _native.KERNEL_VECTOR and info.delta_staging == _native.DELTA_PER_WAVE
    assert info.block_threads == 256 and info.grid_x == 32768 // 4
    assert info.layers_per_wave == 2 and info.grid_y == 1  # capped by the two layers of the CPU pool
    # By default the deltas of streamed rows are staged: the two layers' groups
    # x 16 chunk-waves per workgroup.
    args.delta_staging = _native.DELTA_AUTO
    assert _native.kv_link_describe(args).delta_staging == _native.DELTA_PER_WAVE
    args.stream_source_rows = 1
    info = _native.kv_link_describe(args)
    assert info.delta_staging == _native.DELTA_WORKGROUP
    assert info.block_threads == 1024 and info.grid_x == 32768 // 16 and info.layer_groups_per_block == 1
    del keepalive
    # Half rotary stays on the vector kernel; other partial widths fall back to
    # the generic kernel, and forcing the vector kernel on them fails.
    args, keepalive = _cpu_args(rotary_dim=64)
    assert _native.kv_link_describe(args).kernel == _native.KERNEL_VECTOR
    del keepalive
    args, keepalive = _cpu_args(rotary_dim=32)
    assert _native.kv_link_describe(args).kernel == _native.KERNEL_GENERIC
    args.kernel = _native.KERNEL_VECTOR
    with pytest.raises(_native.NativeCallError) as error:
        _native.kv_link_describe(args)
    assert error.value.reason == "unsupported_kernel_for_shape"
    del keepalive


def test_mixed_index_dtypes_use_the_generic_kernel():
    args, keepalive = _cpu_args(source_slots=torch.arange(8, dtype=torch.int32))
    assert _native.kv_link_describe(args).kernel == _native.KERNEL_GENERIC
    args.kernel = _native.KERNEL_VECTOR
    with pytest.raises(_native.NativeCallError) as error:
        _native.kv_link_describe(args)
    assert error.value.reason == "unsupported_kernel_for_shape"
    del keepalive
    args, keepalive = _cpu_args(**{name: torch.arange(8, dtype=torch.int32) for name in (
        "source_slots", "destination_slots", "local_positions", "global_positions")})
    assert _native.kv_link_describe(args).kernel == _native.KERNEL_VECTOR
    del keepalive


def test_small_links_split_layers_across_waves():
    keys = [torch.zeros(8, 4, 128, dtype=torch.bfloat16) for _ in range(28)]
    info = kv_link.describe_link_launch(
        key_buffers=keys, value_buffers=keys, source_slots=torch.arange(2048),
        destination_slots=torch.arange(2048), local_positions=torch.arange(2048),
        global_positions=torch.arange(2048), cos_sin_cache=build_cos_sin_cache(8, 128),
        prefix_token_count=0, rotary_dim=128, is_neox_style=True,
    )
    assert info["kernel"] == "vector"
    # Layer groups across the grid (per-wave deltas) or within a workgroup (staged).
    groups = info["grid_y"] * info["layer_groups_per_block"]
    assert groups * info["layers_per_wave"] >= 28 and groups > 1


def _describe(layers, heads, dim, tokens, **options):
    keys = [torch.zeros(8, heads, dim, dtype=torch.bfloat16) for _ in range(layers)]
    index = torch.arange(tokens)
    return kv_link.describe_link_launch(
        key_buffers=keys, value_buffers=keys, source_slots=index, destination_slots=index,
        local_positions=index, global_positions=index, cos_sin_cache=build_cos_sin_cache(8, dim),
        prefix_token_count=0, rotary_dim=dim, is_neox_style=True, **options)


@pytest.mark.parametrize("layers,heads,dim,lpw,groups,threads", [
    (28, 4, 128, 0, 7, 14 * 64),    # Qwen2.5-7B: 7 groups of 4 layers x 2 tokens
    (28, 4, 128, 2, 14, 14 * 64),   # 14 groups x 1 token
    (28, 4, 128, 1, 14, 14 * 64),   # 28 groups would exceed 16 waves: 2 layers per wave
    (64, 8, 128, 0, 16, 16 * 64),   # Qwen3-32B: 16 groups x 1 wave (half a token)
    (28, 1, 128, 0, 7, 14 * 64),    # one head: 4 tokens per wave, 2 waves fit the LDS table
    (3, 2, 64, 0, 2, 8 * 64),       # a small link splits its 3 layers in 2 groups; 16-chunk rows:
                                    # 4 chunk-waves (17 tokens) fill the LDS table
])
def test_workgroup_staged_launch_shape(layers, heads, dim, lpw, groups, threads):
    info = _describe(layers, heads, dim, 32768, layers_per_wave=lpw, delta_staging="workgroup")
    assert info["delta_staging"] == "workgroup"
    assert info["layer_groups_per_block"] == groups and info["grid_y"] == 1
    assert info["block_threads"] == threads
    chunk_waves = threads // 64 // groups
    tokens_per_block = -(-chunk_waves * 64 // (heads * dim // 8)) + 1
    assert tokens_per_block <= 18  # the kernel's LDS table
    assert info["grid_x"] == -(-(32768 * heads * dim // 8 // 64) // chunk_waves)


def test_workgroup_staging_falls_back_to_per_wave_deltas():
    # GPT-J pairs and bf16 tables keep per-wave deltas, and so does an explicit
    # layer_groups_per_block; the default stages streamed rows where it fits.
    assert _describe(28, 4, 128, 4096)["delta_staging"] == "per_wave"
    keys = [torch.zeros(8, 4, 128, dtype=torch.bfloat16) for _ in range(4)]
    index = torch.arange(64)
    common = dict(key_buffers=keys, value_buffers=keys, source_slots=index, destination_slots=index,
                  local_positions=index, global_positions=index, prefix_token_count=0, rotary_dim=128,
                  delta_staging="workgroup")
    assert kv_link.describe_link_launch(cos_sin_cache=build_cos_sin_cache(8, 128), is_neox_style=False,
                                        **common)["delta_staging"] == "per_wave"
    assert kv_link.describe_link_launch(cos_sin_cache=build_cos_sin_cache(8, 128).bfloat16(),
                                        is_neox_style=True, **common)["delta_staging"] == "per_wave"
    with pytest.raises(_native.NativeCallError, match="layer_groups_per_block"):
        kv_link.describe_link_launch(cos_sin_cache=build_cos_sin_cache(8, 128), is_neox_style=True,
                                     layer_groups_per_block=2, **common)


def test_cpu_tensors_are_not_eligible():
    keys = torch.zeros(16, 2, 8, dtype=torch.bfloat16)
    result = kv_link.check_fused_kv_link_eligibility(
        key_buffer=keys, value_buffer=keys, source_slots=torch.arange(2),
        destination_slots=torch.arange(2, 4), local_positions=torch.arange(2),
        global_positions=torch.arange(2), cos_sin_cache=build_cos_sin_cache(8, 8), rotary_dim=8,
    )
    assert result == kv_link.LegoLinkFusionEligibility(False, "cuda_tensors_required")


def test_launch_config_resolution_follows_the_reference_rules(monkeypatch):
    config = kv_link.resolve_fused_kv_launch_config(work_items=768)
    assert (config.block_size, config.num_warps, config.num_stages) == (256, 4, 2)
    monkeypatch.setenv("SGLANG_PIC_TRITON_NUM_WARPS", "8")
    config = kv_link.resolve_fused_kv_launch_config(work_items=768)
    assert config.num_warps == 8 and config.source == "explicit_or_environment_override"
    with pytest.raises(ValueError, match="power of two"):
        kv_link.resolve_fused_kv_launch_config(work_items=768, block_size=96)
    with pytest.raises(ValueError, match="num_warps"):
        kv_link.resolve_fused_kv_launch_config(work_items=768, num_warps=3)
    with pytest.raises(ValueError, match="num_stages"):
        kv_link.resolve_fused_kv_launch_config(work_items=768, num_stages=0)


def test_traffic_model_matches_the_reference_formula():
    # Qwen2.5-7B row: 4 heads x 128 dims x 2 bytes = 1024 bytes for K and for V.
    traffic = kv_link.estimate_kv_traffic_bytes(token_count=32768, key_row_bytes=1024,
                                                value_row_bytes=1024, remapped_token_count=30000,
                                                repair_token_count=240)
    copied = 32768 - 240
    assert traffic["triton_lower_bound_bytes"] == 2 * copied * 2048
    assert traffic["torch_lower_bound_bytes"] == 2 * (2 * 32768 * 2048 + 30000 * 1024)
    assert traffic["copied_token_count"] == copied
