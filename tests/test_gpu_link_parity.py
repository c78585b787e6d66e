"""GPU parity of the HIP link and repair-row scatter against the CPU oracle.

Bar: bit-exact on every element (V and copied K are bit copies; re-rotated K
follows the chosen rounding -- the reference's fused kernel or its torch path
-- exactly, which for the fused rounding implies <= 1 bf16 ulp of the exact
rotation).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from legolink_amd import _native, kv_link
from legolink_amd.rope import build_cos_sin_cache
from legolink_amd.workloads import make_workload
from oracle import kv_link_oracle as ko
from tests import rope_math
from tests.gpu_helpers import TORCH_TO_CODE, bits, cache_host, check_workload, make_pool, report

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
AUTO, VECTOR, GENERIC = _native.KERNEL_AUTO, _native.KERNEL_VECTOR, _native.KERNEL_GENERIC

# name, kv dtype, cache dtype, heads, key dim, value dim, rotary dim, neox, kernel, index dtype,
# prefix, mask fraction, layers, tokens, expected kernel
CASES = [
    ("qwen7b_vec", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO, torch.int64, 0, 0.0, 3, 200, "vector"),
    ("qwen7b_vec_prefix_mask", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO, torch.int64, 37, 0.2, 3, 200, "vector"),
    ("qwen7b_generic_prefix_mask", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, GENERIC, torch.int64, 37, 0.2, 3, 200, "generic"),
    ("qwen3_32b_heads8", torch.bfloat16, torch.float32, 8, 128, 128, 128, True, VECTOR, torch.int64, 5, 0.1, 2, 150, "vector"),
    ("tp_shard_one_head_int32", torch.bfloat16, torch.float32, 1, 128, 128, 128, True, AUTO, torch.int32, 3, 0.1, 3, 333, "vector"),
    ("three_heads_straddling_waves", torch.bfloat16, torch.float32, 3, 128, 128, 128, True, AUTO, torch.int64, 0, 0.1, 2, 171, "vector"),
    ("head_dim_64", torch.bfloat16, torch.float32, 2, 64, 64, 64, True, AUTO, torch.int64, 0, 0.1, 2, 190, "vector"),
    ("head_dim_256", torch.bfloat16, torch.float32, 2, 256, 256, 256, True, AUTO, torch.int64, 0, 0.1, 2, 90, "vector"),
    ("head_dim_32", torch.bfloat16, torch.float32, 4, 32, 32, 32, True, AUTO, torch.int64, 0, 0.1, 2, 150, "vector"),
    ("gptj_vec", torch.bfloat16, torch.float32, 4, 128, 128, 128, False, AUTO, torch.int64, 10, 0.1, 2, 150, "vector"),
    ("gptj_generic", torch.bfloat16, torch.float32, 4, 128, 128, 128, False, GENERIC, torch.int64, 10, 0.1, 2, 150, "generic"),
    ("fp16_vec", torch.float16, torch.float32, 4, 128, 128, 128, True, AUTO, torch.int64, 0, 0.1, 2, 150, "vector"),
    ("fp16_generic", torch.float16, torch.float32, 4, 128, 128, 128, True, GENERIC, torch.int64, 0, 0.1, 2, 150, "generic"),
    ("fp16_gptj_d64", torch.float16, torch.float32, 2, 64, 64, 64, False, AUTO, torch.int32, 0, 0.1, 2, 150, "vector"),
    # 16-bit cos/sin tables: widened exactly to fp32, then the same arithmetic.
    ("bf16_key_bf16_cache", torch.bfloat16, torch.bfloat16, 4, 128, 128, 128, True, AUTO, torch.int64, 4, 0.1, 2, 150, "vector"),
    ("bf16_key_fp16_cache", torch.bfloat16, torch.float16, 4, 128, 128, 128, True, AUTO, torch.int64, 4, 0.1, 2, 150, "vector"),
    ("fp16_key_bf16_cache", torch.float16, torch.bfloat16, 4, 128, 128, 128, True, AUTO, torch.int64, 4, 0.1, 2, 150, "vector"),
    ("bf16_cache_gptj_d64", torch.bfloat16, torch.bfloat16, 2, 64, 64, 64, False, AUTO, torch.int32, 3, 0.1, 2, 150, "vector"),
    ("fp16_cache_d256", torch.bfloat16, torch.float16, 2, 256, 256, 256, True, AUTO, torch.int64, 0, 0.1, 2, 90, "vector"),
    ("bf16_cache_gptj_d32", torch.float16, torch.bfloat16, 4, 32, 32, 32, False, AUTO, torch.int64, 2, 0.1, 2, 150, "vector"),
    ("bf16_key_bf16_cache_generic", torch.bfloat16, torch.bfloat16, 4, 128, 128, 128, True, GENERIC, torch.int64, 4, 0.1, 2, 150, "generic"),
    ("fp16_key_fp16_cache_generic", torch.float16, torch.float16, 4, 128, 128, 128, False, GENERIC, torch.int64, 4, 0.1, 2, 150, "generic"),
    # Half rotary (dims past rotary_dim copied): the vector kernel; other partial widths: generic.
    ("partial_rotary", torch.bfloat16, torch.float32, 4, 128, 128, 64, True, AUTO, torch.int64, 0, 0.1, 2, 150, "vector"),
    ("half_rotary_gptj_bf16_cache", torch.bfloat16, torch.bfloat16, 2, 128, 128, 64, False, AUTO, torch.int32, 3, 0.1, 2, 150, "vector"),
    ("half_rotary_d32_fp16", torch.float16, torch.float32, 4, 32, 32, 16, True, AUTO, torch.int64, 2, 0.1, 2, 150, "vector"),
    ("half_rotary_d256_gptj", torch.bfloat16, torch.float16, 2, 256, 256, 128, False, VECTOR, torch.int64, 0, 0.1, 2, 90, "vector"),
    ("partial_rotary_generic", torch.bfloat16, torch.float32, 4, 128, 128, 64, True, GENERIC, torch.int64, 0, 0.1, 2, 150, "generic"),
    ("quarter_rotary", torch.bfloat16, torch.float32, 4, 128, 128, 32, True, AUTO, torch.int64, 0, 0.1, 2, 150, "generic"),
    ("value_dim_differs", torch.bfloat16, torch.float32, 2, 128, 64, 128, True, AUTO, torch.int64, 0, 0.1, 2, 150, "generic"),
    ("odd_dims_gptj", torch.bfloat16, torch.float32, 3, 40, 24, 16, False, AUTO, torch.int64, 2, 0.1, 2, 150, "generic"),
    ("prefix_is_everything", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO, torch.int64, 150, 0.0, 2, 150, "vector"),
    ("all_masked", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO, torch.int64, 0, 1.0, 2, 150, "vector"),
    ("single_token", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO, torch.int64, 0, 0.0, 2, 1, "vector"),
    ("seventy_layers", torch.bfloat16, torch.float32, 2, 128, 128, 128, True, AUTO, torch.int64, 3, 0.1, 70, 64, "vector"),
    # The vector kernel reads all four maps with one index type; a mix goes to the generic kernel.
    ("mixed_index_dtypes", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO,
     (torch.int32, torch.int64, torch.int64, torch.int32), 6, 0.1, 3, 200, "generic"),
    ("five_layers_odd_tail", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO, torch.int32, 2, 0.1, 5, 129, "vector"),
]


def _corrupt(rng, fraction, src, dst, local, global_, slots, cache_rows):
    """Plant out-of-range slots and positions in about ``fraction`` of the tokens."""

    src, dst, local, global_ = (a.copy() for a in (src, dst, local, global_))
    for t in np.flatnonzero(rng.random(src.shape[0]) < fraction):
        kind = int(rng.integers(0, 8))
        target = (src, dst, local, global_)[kind % 4]
        limit = slots if kind % 4 < 2 else cache_rows
        target[t] = -1 - int(rng.integers(0, 3)) if kind < 4 else limit + int(rng.integers(0, 3))
    return src, dst, local, global_


def _run_case(device, case, *, seed=11, mask_dtype=torch.uint8, cache_layout="dense", rounding="fused",
              corrupt=0.0, **link_options):
    (name, dtype, cache_dtype, heads, kdim, vdim, rotary, neox, kernel, index_dtype, prefix,
     mask_fraction, layers, tokens, expected_kernel) = case
    report(f"case {name}: layers={layers} heads={heads} kdim={kdim} vdim={vdim} rotary={rotary} "
           f"neox={neox} tokens={tokens} kernel={kernel} rounding={rounding}")
    slots = 2 * tokens + 41
    rng = np.random.default_rng(seed)
    perm = rng.permutation(slots)
    src_np, dst_np = perm[:tokens], perm[tokens : 2 * tokens]
    max_position = 70_000
    local_np = rng.integers(0, max_position, size=tokens)
    global_np = rng.integers(0, max_position, size=tokens)
    mask_np = (rng.random(tokens) < mask_fraction).astype(np.uint8)
    skipped = None
    if corrupt:
        src_np, dst_np, local_np, global_np = _corrupt(rng, corrupt, src_np, dst_np, local_np, global_np,
                                                       slots, max_position)
        skipped = torch.zeros(1, dtype=torch.int64, device=device)
        link_options = {**link_options, "skipped_rows": skipped}
    keys, values = make_pool(layers, slots, heads, kdim, vdim, dtype, device, seed)
    table = build_cos_sin_cache(max_position, rotary, theta=1e6).to(cache_dtype)
    if cache_layout == "strided":
        wide = torch.zeros(max_position, 2 * rotary + 4, dtype=cache_dtype)
        wide[:, 1 : 1 + 2 * rotary : 2] = table
        table_dev = wide.to(device)[:, 1 : 1 + 2 * rotary : 2]
        assert table_dev.stride(1) == 2
    else:
        table_dev = table.to(device)
    index_dtypes = index_dtype if isinstance(index_dtype, tuple) else (index_dtype,) * 4
    maps = [torch.from_numpy(a).to(d).to(device)
            for a, d in zip((src_np, dst_np, local_np, global_np), index_dtypes)]
    mask = torch.from_numpy(mask_np).to(device).to(mask_dtype) if mask_fraction > 0 else None
    key_np = [bits(k) for k in keys]
    value_np = [bits(v) for v in values]
    expected_k, expected_v = ko.link_pool(
        key_np, value_np, src_np, dst_np, local_np, global_np, cache_host(table),
        key_dtype=TORCH_TO_CODE[dtype], cache_dtype=TORCH_TO_CODE[cache_dtype],
        rotary_dim=rotary, neox=neox, prefix=prefix, repair_mask=mask_np if mask is not None else None,
        rounding=ko.EAGER if rounding == "eager" else ko.FUSED,
    )
    describe_options = {key: value for key, value in link_options.items() if key != "skipped_rows"}
    launch = kv_link.describe_link_launch(
        key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
        local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table_dev,
        prefix_token_count=prefix, rotary_dim=rotary, is_neox_style=neox, repair_mask=mask,
        kernel=kernel, **describe_options,
    )
    assert launch["kernel"] == expected_kernel, launch
    if link_options.get("delta_staging") in ("workgroup", "table"):
        assert launch["delta_staging"] == link_options["delta_staging"], launch
    kv_link.fused_kv_link_layers_inplace(
        key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
        local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table_dev,
        prefix_token_count=prefix, rotary_dim=rotary, is_neox_style=neox, repair_mask=mask,
        kernel=kernel, rounding=rounding, **link_options,
    )
    torch.cuda.synchronize(device)
    for layer in range(layers):
        got_k, got_v = bits(keys[layer]), bits(values[layer])
        if dtype == torch.float16:
            # NaN payloads are not part of the contract; inputs here hold none.
            assert not np.isnan(got_k.view(np.float16)).any()
        assert np.array_equal(got_v, expected_v[layer]), f"{name}: V layer {layer}"
        diff = np.argwhere(got_k != expected_k[layer])
        assert diff.size == 0, f"{name}: K layer {layer} differs at {diff[:5].tolist()}"
    if skipped is not None:
        expected_skips = ko.skipped_token_mask(
            src_np, dst_np, local_np, global_np, source_slots=slots, destination_slots=slots,
            cache_rows=max_position, prefix=prefix, repair_mask=mask_np if mask is not None else None)
        assert expected_skips.any(), f"{name}: no token was corrupted"
        assert int(skipped.item()) == int(expected_skips.sum()), f"{name}: skipped-row count"


@pytest.mark.parametrize("case", CASES, ids=[case[0] for case in CASES])
def test_link_matches_oracle(gpu_device, case):
    _run_case(gpu_device, case)


# Workgroup-staged deltas (neox, full rotary, fp32 table): name, kv dtype, heads, dim,
# layers, tokens, prefix, mask fraction, layers per wave, index dtype.
STAGED_CASES = [
    ("qwen7b_28_layers", torch.bfloat16, 4, 128, 28, 301, 17, 0.1, 0, torch.int64),
    ("qwen7b_two_layers_per_wave", torch.bfloat16, 4, 128, 28, 130, 0, 0.1, 2, torch.int32),
    ("one_layer_per_wave_raised", torch.bfloat16, 4, 128, 28, 70, 3, 0.0, 1, torch.int64),
    ("qwen3_32b_64_layers", torch.bfloat16, 8, 128, 64, 90, 5, 0.1, 0, torch.int64),
    ("seventy_layers_two_launches", torch.bfloat16, 2, 128, 70, 64, 3, 0.1, 0, torch.int64),
    ("one_head_four_tokens_per_wave", torch.bfloat16, 1, 128, 28, 333, 6, 0.1, 0, torch.int32),
    ("head_dim_256", torch.bfloat16, 2, 256, 5, 150, 0, 0.1, 0, torch.int64),
    ("head_dim_64_fp16", torch.float16, 4, 64, 7, 171, 9, 0.1, 0, torch.int64),
    ("head_dim_32_small_link", torch.bfloat16, 4, 32, 3, 45, 2, 0.1, 0, torch.int64),
    ("single_token", torch.bfloat16, 4, 128, 28, 1, 0, 0.0, 0, torch.int64),
    ("prefix_is_everything", torch.bfloat16, 4, 128, 6, 100, 100, 0.0, 0, torch.int64),
]


@pytest.mark.parametrize("rounding", ["fused", "eager"])
@pytest.mark.parametrize("staged", STAGED_CASES, ids=[case[0] for case in STAGED_CASES])
def test_workgroup_staged_deltas_match_oracle(gpu_device, staged, rounding):
    name, dtype, heads, dim, layers, tokens, prefix, mask_fraction, lpw, index_dtype = staged
    case = (name, dtype, torch.float32, heads, dim, dim, dim, True, AUTO, index_dtype, prefix,
            mask_fraction, layers, tokens, "vector")
    _run_case(gpu_device, case, rounding=rounding, delta_staging="workgroup", layers_per_wave=lpw)


# The delta table and the layer-major walk (neox, full rotary, fp32 table,
# rows of whole KiB): name, kv dtype, heads, dim, layers, tokens (odd counts
# leave the last wave one token), prefix (even and odd, so that it ends inside
# a wave's token pair), mask fraction, index dtype, source pool.
TABLE_CASES = [
    ("qwen7b_28_layers", torch.bfloat16, 4, 128, 28, 301, 17, 0.1, torch.int64, "own"),
    ("qwen7b_even_prefix", torch.bfloat16, 4, 128, 28, 300, 40, 0.0, torch.int32, "own"),
    ("qwen3_32b_two_parts_per_row", torch.bfloat16, 8, 128, 64, 91, 5, 0.1, torch.int64, "own"),
    ("seventy_layers_two_launches", torch.bfloat16, 4, 128, 70, 63, 3, 0.1, torch.int64, "own"),
    ("head_dim_64", torch.float16, 8, 64, 7, 171, 9, 0.1, torch.int64, "own"),
    ("head_dim_256", torch.bfloat16, 2, 256, 5, 150, 0, 0.1, torch.int32, "own"),
    ("head_dim_32", torch.bfloat16, 16, 32, 3, 45, 2, 0.1, torch.int64, "own"),
    ("single_token", torch.bfloat16, 4, 128, 28, 1, 0, 0.0, torch.int64, "own"),
    ("prefix_is_everything", torch.bfloat16, 4, 128, 6, 100, 100, 0.0, torch.int64, "own"),
    ("separate_source_pool", torch.bfloat16, 4, 128, 6, 257, 30, 0.1, torch.int64, "separate"),
]


@pytest.mark.parametrize("rounding", ["fused", "eager"])
@pytest.mark.parametrize("table_case", TABLE_CASES, ids=[case[0] for case in TABLE_CASES])
def test_delta_table_layer_major_link_matches_oracle(gpu_device, table_case, rounding):
    name, dtype, heads, dim, layers, tokens, prefix, mask_fraction, index_dtype, source = table_case
    case = (name, dtype, torch.float32, heads, dim, dim, dim, True, AUTO, index_dtype, prefix,
            mask_fraction, layers, tokens, "vector")
    workspace = torch.empty(kv_link.delta_workspace_bytes(tokens, dim) // 4 + 1, dtype=torch.float32,
                            device=gpu_device)
    options = {"delta_staging": "table", "delta_workspace": workspace}
    if source == "separate":
        _run_separate_source_case(gpu_device, case, rounding=rounding, **options)
    else:
        _run_case(gpu_device, case, rounding=rounding, **options)


def test_delta_table_without_workspace_falls_back_to_staging(gpu_device):
    keys, values = make_pool(2, 64, 4, 128, 128, torch.bfloat16, gpu_device, 1)
    maps = [torch.arange(10, device=gpu_device), torch.arange(20, 30, device=gpu_device),
            torch.arange(10, device=gpu_device), torch.arange(10, device=gpu_device) + 3]
    table = build_cos_sin_cache(64, 128).to(gpu_device)
    common = dict(key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
                  local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table, prefix_token_count=0,
                  rotary_dim=128, is_neox_style=True, delta_staging="table", stream_source_rows=True)
    assert kv_link.describe_link_launch(**common)["delta_staging"] == "workgroup"
    small = torch.empty(10 * 128 - 1, dtype=torch.float32, device=gpu_device)  # one entry short
    assert kv_link.describe_link_launch(**common, delta_workspace=small)["delta_staging"] == "workgroup"
    enough = torch.empty(10 * 128, dtype=torch.float32, device=gpu_device)
    launch = kv_link.describe_link_launch(**common, delta_workspace=enough)
    assert launch["delta_staging"] == "table" and launch["block_threads"] == 256


def _run_separate_source_case(device, case, *, rounding, **link_options):
    """A link whose sources live in a second pool of the same row layout
    (the snapshot arena's case), through the delta table."""

    (name, dtype, _, heads, dim, _, rotary, _, _, index_dtype, prefix, mask_fraction, layers, tokens, _) = case
    report(f"table case {name}: separate source pool, rounding={rounding}")
    rng = np.random.default_rng(41)
    slots, arena_slots = 2 * tokens + 9, tokens + 5
    keys, values = make_pool(layers, slots, heads, dim, dim, dtype, device, 41)
    arena_k, arena_v = make_pool(layers, arena_slots, heads, dim, dim, dtype, device, 42)
    src_np = rng.permutation(arena_slots)[:tokens]
    dst_np = rng.permutation(slots)[:tokens]
    local_np = rng.integers(0, 9000, size=tokens)
    global_np = rng.integers(0, 9000, size=tokens)
    mask_np = (rng.random(tokens) < mask_fraction).astype(np.uint8)
    table = build_cos_sin_cache(9000, rotary, theta=1e6)
    expected_k, expected_v = ko.link_pool(
        [bits(k) for k in keys], [bits(v) for v in values], src_np, dst_np, local_np, global_np, table.numpy(),
        key_dtype=TORCH_TO_CODE[dtype], cache_dtype=ko.F32, rotary_dim=rotary, neox=True, prefix=prefix,
        repair_mask=mask_np, source_key_layers=[bits(k) for k in arena_k],
        source_value_layers=[bits(v) for v in arena_v], rounding=ko.EAGER if rounding == "eager" else ko.FUSED)
    maps = [torch.from_numpy(a).to(index_dtype).to(device) for a in (src_np, dst_np, local_np, global_np)]
    kv_link.fused_kv_link_layers_inplace(
        key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
        local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table.to(device),
        prefix_token_count=prefix, rotary_dim=rotary, is_neox_style=True,
        repair_mask=torch.from_numpy(mask_np).to(device), source_key_buffers=arena_k,
        source_value_buffers=arena_v, rounding=rounding, **link_options)
    torch.cuda.synchronize(device)
    for layer in range(layers):
        assert np.array_equal(bits(keys[layer]), expected_k[layer]), f"{name}: K layer {layer}"
        assert np.array_equal(bits(values[layer]), expected_v[layer]), f"{name}: V layer {layer}"


@pytest.mark.parametrize("table_case", TABLE_CASES[:4], ids=[case[0] for case in TABLE_CASES[:4]])
def test_out_of_range_tokens_are_counted_with_the_delta_table(gpu_device, table_case):
    name, dtype, heads, dim, layers, tokens, prefix, mask_fraction, index_dtype, _ = table_case
    case = (name, dtype, torch.float32, heads, dim, dim, dim, True, AUTO, index_dtype, prefix,
            mask_fraction, layers, tokens, "vector")
    workspace = torch.empty(kv_link.delta_workspace_bytes(tokens, dim), dtype=torch.uint8, device=gpu_device)
    _run_case(gpu_device, case, delta_staging="table", delta_workspace=workspace, corrupt=0.15, seed=31)


SKIP_CASES = [case for case in CASES if case[0] in {
    "qwen7b_vec", "qwen7b_vec_prefix_mask", "qwen7b_generic_prefix_mask", "tp_shard_one_head_int32",
    "gptj_vec", "fp16_generic", "bf16_key_bf16_cache", "partial_rotary_generic", "seventy_layers",
    "mixed_index_dtypes", "five_layers_odd_tail"}]


@pytest.mark.parametrize("case", SKIP_CASES, ids=[case[0] for case in SKIP_CASES])
def test_out_of_range_tokens_are_skipped_and_counted(gpu_device, case):
    """Tokens with a slot or position out of range store nothing and are
    counted once per call (over several launches too: seventy_layers)."""

    _run_case(gpu_device, case, corrupt=0.15, seed=23)


@pytest.mark.parametrize("staged", STAGED_CASES[:5], ids=[case[0] for case in STAGED_CASES[:5]])
def test_out_of_range_tokens_are_counted_with_staged_deltas(gpu_device, staged):
    name, dtype, heads, dim, layers, tokens, prefix, mask_fraction, lpw, index_dtype = staged
    case = (name, dtype, torch.float32, heads, dim, dim, dim, True, AUTO, index_dtype, prefix,
            mask_fraction, layers, tokens, "vector")
    _run_case(gpu_device, case, delta_staging="workgroup", layers_per_wave=lpw, corrupt=0.15, seed=29,
              rounding="eager")


@pytest.mark.parametrize("case", CASES, ids=[case[0] for case in CASES])
def test_eager_link_matches_oracle(gpu_device, case):
    """The torch path's rounding points (pic_runtime.py:6025-6058) on every shape."""

    _run_case(gpu_device, case, rounding="eager")


def test_bool_mask_and_strided_cache(gpu_device):
    case = ("bool_mask_strided_cache", torch.bfloat16, torch.float32, 4, 128, 128, 128, True, AUTO,
            torch.int64, 7, 0.3, 2, 160, "generic")
    _run_case(gpu_device, case, mask_dtype=torch.bool, cache_layout="strided")


def test_per_layer_entry_equals_all_layer_entry(gpu_device):
    layers, slots, tokens = 4, 700, 300
    rng = np.random.default_rng(3)
    perm = rng.permutation(slots)
    src = torch.from_numpy(perm[:tokens]).to(gpu_device)
    dst = torch.from_numpy(perm[tokens : 2 * tokens]).to(gpu_device)
    local = torch.from_numpy(rng.integers(0, 4096, size=tokens)).to(gpu_device)
    glob = torch.from_numpy(rng.integers(0, 4096, size=tokens)).to(gpu_device)
    table = build_cos_sin_cache(4096, 128).to(gpu_device)
    keys_a, values_a = make_pool(layers, slots, 4, 128, 128, torch.bfloat16, gpu_device, 5)
    keys_b = [k.clone() for k in keys_a]
    values_b = [v.clone() for v in values_a]
    for key, value in zip(keys_a, values_a):
        kv_link.fused_kv_link_inplace(
            key_buffer=key, value_buffer=value, source_slots=src, destination_slots=dst,
            local_positions=local, global_positions=glob, cos_sin_cache=table,
            prefix_token_count=11, rotary_dim=128, is_neox_style=True,
        )
    kv_link.fused_kv_link_layers_inplace(
        key_buffers=keys_b, value_buffers=values_b, source_slots=src, destination_slots=dst,
        local_positions=local, global_positions=glob, cos_sin_cache=table,
        prefix_token_count=11, rotary_dim=128, is_neox_style=True,
    )
    torch.cuda.synchronize(gpu_device)
    for a, b in zip(keys_a + values_a, keys_b + values_b):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_out_of_range_rows_are_skipped_or_rejected(gpu_device):
    slots, tokens = 100, 40
    keys, values = make_pool(2, slots, 4, 128, 128, torch.bfloat16, gpu_device, 9)
    rng = np.random.default_rng(9)
    perm = rng.permutation(slots)
    src_np, dst_np = perm[:tokens].copy(), perm[tokens : 2 * tokens].copy()
    local_np = rng.integers(0, 512, size=tokens)
    global_np = rng.integers(0, 512, size=tokens)
    src_np[3] = slots + 5          # source outside the pool
    dst_np[7] = -1                 # negative destination
    global_np[11] = 512            # position outside the table
    table = build_cos_sin_cache(512, 128)
    bad = {3, 7, 11}
    good = np.array([t for t in range(tokens) if t not in bad])
    expected_k, expected_v = ko.link_pool(
        [bits(k) for k in keys], [bits(v) for v in values], src_np[good], dst_np[good],
        local_np[good], global_np[good], table.numpy(), key_dtype=ko.BF16, cache_dtype=ko.F32,
        rotary_dim=128, neox=True, prefix=0,
    )
    maps = [torch.from_numpy(a).to(gpu_device) for a in (src_np, dst_np, local_np, global_np)]
    with pytest.raises(IndexError):
        kv_link.fused_kv_link_layers_inplace(
            key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
            local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table.to(gpu_device),
            prefix_token_count=0, rotary_dim=128, is_neox_style=True, validate_indices=True,
        )
    kv_link.fused_kv_link_layers_inplace(
        key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
        local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table.to(gpu_device),
        prefix_token_count=0, rotary_dim=128, is_neox_style=True,
    )
    torch.cuda.synchronize(gpu_device)
    for layer in range(2):
        assert np.array_equal(bits(keys[layer]), expected_k[layer])
        assert np.array_equal(bits(values[layer]), expected_v[layer])


def test_reference_relocation_case(gpu_device):
    """tests/pic/test_kv_relocation.py:47-103 on the HIP op: bit-exact against the
    oracle and within the reference's own atol 2e-2 of the fp64 relocation."""

    case = GOLDEN["kv_relocation"]
    slots, heads, rotary = case["gpu_pool_slots"], case["heads"], case["rotary_dim"]
    generator = torch.Generator(device=gpu_device).manual_seed(20260824)
    key = torch.randn(slots, heads, rotary, device=gpu_device, dtype=torch.bfloat16, generator=generator)
    value = torch.randn(slots, heads, rotary, device=gpu_device, dtype=torch.bfloat16, generator=generator)
    source = torch.tensor(case["source_slots"], device=gpu_device)
    destination = torch.tensor(case["gpu_destination"], device=gpu_device)
    local = torch.tensor(case["local"], device=gpu_device)
    glob = torch.tensor(case["global"], device=gpu_device)
    table = build_cos_sin_cache(16, rotary, theta=10_000.0)
    # Source rows hold K rotated to their local positions (compile-time keys).
    raw = key[source].float().cpu().numpy().astype(np.float64)
    compiled = rope_math.rotate(raw, np.array(case["local"]), rotary, theta=10_000.0)
    key[source] = torch.from_numpy(compiled).to(torch.bfloat16).to(gpu_device)
    key_before, value_before = bits(key), bits(value)
    expected_k, expected_v = ko.link_pool(
        [key_before], [value_before], np.array(case["source_slots"]), np.array(case["gpu_destination"]),
        np.array(case["local"]), np.array(case["global"]), table.numpy(), key_dtype=ko.BF16,
        cache_dtype=ko.F32, rotary_dim=rotary, neox=True, prefix=0,
    )
    kv_link.fused_kv_link_inplace(
        key_buffer=key, value_buffer=value, source_slots=source, destination_slots=destination,
        local_positions=local, global_positions=glob, cos_sin_cache=table.to(gpu_device),
        prefix_token_count=0, rotary_dim=rotary, is_neox_style=True,
    )
    torch.cuda.synchronize(gpu_device)
    assert np.array_equal(bits(key), expected_k[0])
    assert np.array_equal(bits(value), expected_v[0])
    # The re-rotated keys are the raw keys rotated straight to the global positions.
    truth = rope_math.rotate(raw, np.array(case["global"]), rotary, theta=10_000.0)
    got = key[destination].float().cpu().numpy()
    atol = case["gpu_atol"]
    assert np.all(np.abs(got - truth) <= atol + atol * np.abs(truth))


def test_repair_writeback_cases(gpu_device):
    """tests/pic/test_kv_writeback.py:12-55 through the HIP scatter (bf16 pools)."""

    single = GOLDEN["repair_writeback"]["single"]
    generator = torch.Generator(device=gpu_device).manual_seed(20260824)
    shape = (single["pool_slots"], single["heads"], single["head_dim"])
    key = torch.randn(*shape, device=gpu_device, dtype=torch.bfloat16, generator=generator)
    value = torch.randn(*shape, device=gpu_device, dtype=torch.bfloat16, generator=generator)
    dest = torch.tensor(single["destination"], device=gpu_device)
    rk = torch.randn(len(single["destination"]), *shape[1:], device=gpu_device, dtype=torch.bfloat16, generator=generator)
    rv = torch.randn_like(rk)
    key_before, value_before = bits(key), bits(value)
    ek, ev = ko.scatter_rows([key_before], [value_before], np.array(single["destination"]),
                             bits(rk)[None], bits(rv)[None])
    kv_link.scatter_kv_rows_inplace(key_buffers=[key], value_buffers=[value], destination_slots=dest,
                                    repaired_keys=rk, repaired_values=rv)
    torch.cuda.synchronize(gpu_device)
    assert np.array_equal(bits(key), ek[0]) and np.array_equal(bits(value), ev[0])
    source = np.array(single["source_slots"])
    assert np.array_equal(bits(key)[source], key_before[source])
    assert np.array_equal(bits(value)[source], value_before[source])

    multi = GOLDEN["repair_writeback"]["multi"]
    key = torch.zeros(multi["pool_slots"], multi["heads"], multi["head_dim"], device=gpu_device, dtype=torch.bfloat16)
    value = torch.zeros_like(key)
    slots = [s for row in multi["row_slots"] for s in row]
    rk = torch.arange(len(slots) * multi["head_dim"], dtype=torch.float32).view(len(slots), 1, multi["head_dim"]).to(torch.bfloat16).to(gpu_device)
    rv = (rk.float() + multi["value_offset"]).to(torch.bfloat16)
    kv_link.scatter_kv_rows_inplace(key_buffers=[key], value_buffers=[value],
                                    destination_slots=torch.tensor(slots, device=gpu_device),
                                    repaired_keys=rk, repaired_values=rv)
    torch.cuda.synchronize(gpu_device)
    assert torch.equal(key[torch.tensor(slots)], rk)
    assert torch.equal(value[torch.tensor(slots)], rv)
    assert torch.count_nonzero(key[torch.tensor(multi["untouched"])]) == 0


def test_scatter_unaligned_rows_use_the_element_path(gpu_device):
    layers, slots, rows = 3, 64, 10
    keys, values = make_pool(layers, slots, 3, 7, 5, torch.bfloat16, gpu_device, 21)
    dest = torch.randperm(slots, device=gpu_device)[:rows]
    rk = torch.randn(layers, rows, 3, 7, device=gpu_device, dtype=torch.bfloat16)
    rv = torch.randn(layers, rows, 3, 5, device=gpu_device, dtype=torch.bfloat16)
    ek, ev = ko.scatter_rows([bits(k) for k in keys], [bits(v) for v in values], dest.cpu().numpy(),
                             bits(rk), bits(rv))
    kv_link.scatter_kv_rows_inplace(key_buffers=keys, value_buffers=values, destination_slots=dest,
                                    repaired_keys=rk, repaired_values=rv)
    torch.cuda.synchronize(gpu_device)
    for layer in range(layers):
        assert np.array_equal(bits(keys[layer]), ek[layer])
        assert np.array_equal(bits(values[layer]), ev[layer])


def test_eligibility_reasons_on_device(gpu_device):
    keys, values = make_pool(1, 32, 2, 8, 8, torch.bfloat16, gpu_device, 1)
    maps = dict(
        source_slots=torch.arange(4, device=gpu_device),
        destination_slots=torch.arange(4, 8, device=gpu_device),
        local_positions=torch.arange(4, device=gpu_device),
        global_positions=torch.arange(4, 8, device=gpu_device),
    )
    table = build_cos_sin_cache(16, 8).to(gpu_device)

    def reason(**overrides):
        kwargs = dict(key_buffer=keys[0], value_buffer=values[0], cos_sin_cache=table, rotary_dim=8, **maps)
        kwargs.update(overrides)
        return kv_link.check_fused_kv_link_eligibility(**kwargs).reason

    assert reason() == "supported"
    assert reason(key_buffer=keys[0].float()) == "kv_dtype_mismatch"
    assert reason(key_buffer=keys[0].float(), value_buffer=values[0].float()) == "fp16_or_bf16_required"
    assert reason(rotary_dim=7) == "even_rotary_dim_required"
    assert reason(rotary_dim=10) == "rotary_dim_exceeds_head_dim"
    assert reason(source_slots=maps["source_slots"].float()) == "integer_token_maps_required"
    assert reason(repair_mask=torch.zeros(3, dtype=torch.uint8, device=gpu_device)) == "repair_mask_length_mismatch"
    assert reason(cos_sin_cache=table.double()) == "unsupported_cos_sin_dtype"
    assert reason(source_slots=maps["source_slots"][:0]) == "empty_link"
    with pytest.raises(RuntimeError, match="HIP LegoLink fusion is unavailable: even_rotary_dim_required"):
        kv_link.fused_kv_link_inplace(key_buffer=keys[0], value_buffer=values[0], cos_sin_cache=table,
                                      rotary_dim=7, prefix_token_count=0, is_neox_style=True, **maps)
    with pytest.raises(ValueError, match="prefix_token_count is outside"):
        kv_link.fused_kv_link_inplace(key_buffer=keys[0], value_buffer=values[0], cos_sin_cache=table,
                                      rotary_dim=8, prefix_token_count=5, is_neox_style=True, **maps)


@pytest.mark.parametrize("name,sample", [("c1", None), ("c2", None), ("c5", None), ("c4", None), ("c3", 16384)])
def test_full_size_workload(gpu_device, name, sample):
    result = check_workload(make_workload(name), gpu_device, sample_tokens=sample)
    assert result["mismatches"] == 0


def test_full_size_workload_generic_kernel(gpu_device):
    result = check_workload(make_workload("c1"), gpu_device, kernel=GENERIC)
    assert result["mismatches"] == 0


@pytest.mark.parametrize("name", ["c2", "c5", "c4"])
def test_full_size_link_as_benched(gpu_device, name):
    """The exact link bench.py times: the executor with repair rows left out of
    the device-built maps, non-temporal row loads, fused rounding."""

    result = check_workload(make_workload(name), gpu_device, via_executor=True, rounding="fused")
    assert result["mismatches"] == 0
    assert result["launch"]["stream_source_rows"] and result["launch"]["kernel"] == "vector"


def test_full_size_c3_link_as_benched(gpu_device):
    """c3 as bench.py times it: 64 requests through prepare_links (one map
    build, the device sort of the rotated rows by source slot, cacheable row
    loads, per-wave deltas), the write-back of every request's repair rows;
    16,384 sampled tokens compared with the oracle, and every row outside the
    destinations checked unchanged."""

    result = check_workload(make_workload("c3"), gpu_device, sample_tokens=16384, via_executor=True,
                            rounding="fused")
    assert result["mismatches"] == 0
    launch = result["launch"]
    assert launch["kernel"] == "vector" and not launch["stream_source_rows"]
    assert launch["delta_staging"] == "per_wave" and launch["visit_order"] == "source"


@pytest.mark.parametrize("name", ["c2", "c5", "c4"])
def test_full_size_eager_link(gpu_device, name):
    """The reference's default link (fused mode off: its torch path's rounding)
    through the executor at full size."""

    result = check_workload(make_workload(name), gpu_device, via_executor=True, rounding="eager")
    assert result["mismatches"] == 0
    assert result["launch"]["rounding"] == "eager"


def test_full_size_eager_link_generic_kernel(gpu_device):
    result = check_workload(make_workload("c1"), gpu_device, kernel=GENERIC, rounding="eager")
    assert result["mismatches"] == 0


@pytest.mark.parametrize("waves,groups,layers_per_wave", [(4, 2, 2), (4, 4, 1), (4, 4, 3), (8, 8, 1), (2, 2, 4)])
def test_layer_groups_per_block_shapes_match_oracle(gpu_device, waves, groups, layers_per_wave):
    """Blocks whose waves share tokens across layer groups (7 layers, so the last
    group is partial and some waves have no layer) give the same pool."""

    layers, slots, tokens = 7, 900, 300
    rng = np.random.default_rng(17)
    perm = rng.permutation(slots)
    src_np, dst_np = perm[:tokens], perm[tokens : 2 * tokens]
    local_np = rng.integers(0, 4096, size=tokens)
    global_np = rng.integers(0, 4096, size=tokens)
    mask_np = (rng.random(tokens) < 0.1).astype(np.uint8)
    keys, values = make_pool(layers, slots, 4, 128, 128, torch.bfloat16, gpu_device, 17)
    table = build_cos_sin_cache(4096, 128)
    expected_k, expected_v = ko.link_pool(
        [bits(k) for k in keys], [bits(v) for v in values], src_np, dst_np, local_np, global_np,
        table.numpy(), key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=128, neox=True, prefix=9,
        repair_mask=mask_np,
    )
    maps = [torch.from_numpy(a).to(gpu_device) for a in (src_np, dst_np, local_np, global_np, mask_np)]
    link = kv_link.PreparedKVLink(
        key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
        local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table.to(gpu_device),
        prefix_token_count=9, rotary_dim=128, is_neox_style=True, repair_mask=maps[4],
        num_warps=waves, layers_per_wave=layers_per_wave, layer_groups_per_block=groups,
    )
    assert link.launch["layer_groups_per_block"] == groups
    link()
    torch.cuda.synchronize(gpu_device)
    for layer in range(layers):
        assert np.array_equal(bits(keys[layer]), expected_k[layer]), f"K layer {layer}"
        assert np.array_equal(bits(values[layer]), expected_v[layer]), f"V layer {layer}"


def test_streamed_row_loads_give_the_same_pool(gpu_device):
    """stream_source_rows only changes how rows are loaded (non-temporal)."""

    report("streamed vs cached row loads")
    layers, tokens = 3, 400
    rng = np.random.default_rng(77)
    pools = []
    for stream in (False, True):
        keys, values = make_pool(layers, 2048, 4, 128, 128, torch.bfloat16, gpu_device, 77)
        perm = rng.permutation(2048) if not pools else perm
        maps = [torch.from_numpy(a).to(gpu_device) for a in (
            perm[:tokens], perm[tokens:2 * tokens], np.arange(tokens) % 700, np.arange(tokens) + 100)]
        kv_link.fused_kv_link_layers_inplace(
            key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
            local_positions=maps[2], global_positions=maps[3], cos_sin_cache=build_cos_sin_cache(1024, 128).to(gpu_device),
            prefix_token_count=5, rotary_dim=128, is_neox_style=True, kernel=VECTOR, stream_source_rows=stream)
        torch.cuda.synchronize(gpu_device)
        pools.append(([bits(k) for k in keys], [bits(v) for v in values]))
    for layer in range(layers):
        assert np.array_equal(pools[0][0][layer], pools[1][0][layer])
        assert np.array_equal(pools[0][1][layer], pools[1][1][layer])
