"""GPU tests of the separate-source link: clone-mode capture, links that mix
clone and reference blocks, and group promotion."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from legolink_amd import _native, kv_link
from legolink_amd.link_plan import resolve_link_plan
from legolink_amd.link_runtime import KVLinkExecutor, KVPool, SnapshotArena
from legolink_amd.registry import LegoLinkBlockRegistry
from legolink_amd.rope import RotarySpec, build_cos_sin_cache
from oracle import kv_link_oracle as ko
from tests import rope_math
from tests.gpu_helpers import bits, make_pool, report

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kernel", [_native.KERNEL_VECTOR, _native.KERNEL_GENERIC])
def test_link_reads_a_separate_source_pool(gpu_device, kernel):
    report(f"separate source pool, kernel {kernel}")
    layers, tokens = 3, 250
    rng = np.random.default_rng(23)
    keys, values = make_pool(layers, 600, 4, 128, 128, torch.bfloat16, gpu_device, 23)
    src_keys, src_values = make_pool(layers, 400, 4, 128, 128, torch.bfloat16, gpu_device, 24)
    src_np = rng.permutation(400)[:tokens]
    dst_np = rng.permutation(600)[:tokens]
    local_np = rng.integers(0, 3000, size=tokens)
    global_np = rng.integers(0, 3000, size=tokens)
    table = build_cos_sin_cache(3000, 128)
    expected_k, expected_v = ko.link_pool(
        [bits(k) for k in keys], [bits(v) for v in values], src_np, dst_np, local_np, global_np,
        table.numpy(), key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=128, neox=True, prefix=12,
        source_key_layers=[bits(k) for k in src_keys], source_value_layers=[bits(v) for v in src_values],
    )
    before_sources = [bits(k) for k in src_keys]
    maps = [torch.from_numpy(a).to(gpu_device) for a in (src_np, dst_np, local_np, global_np)]
    kv_link.fused_kv_link_layers_inplace(
        key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
        local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table.to(gpu_device),
        prefix_token_count=12, rotary_dim=128, is_neox_style=True, kernel=kernel,
        source_key_buffers=src_keys, source_value_buffers=src_values,
    )
    torch.cuda.synchronize(gpu_device)
    for layer in range(layers):
        assert np.array_equal(bits(keys[layer]), expected_k[layer])
        assert np.array_equal(bits(values[layer]), expected_v[layer])
        assert np.array_equal(bits(src_keys[layer]), before_sources[layer])


def test_source_pool_layout_must_match(gpu_device):
    keys, values = make_pool(1, 64, 4, 128, 128, torch.bfloat16, gpu_device, 1)
    src_keys, src_values = make_pool(1, 64, 2, 128, 128, torch.bfloat16, gpu_device, 2)
    index = torch.arange(4, device=gpu_device)
    with pytest.raises(RuntimeError, match="kv_head_layout_mismatch"):
        kv_link.fused_kv_link_layers_inplace(
            key_buffers=keys, value_buffers=values, source_slots=index, destination_slots=index + 8,
            local_positions=index, global_positions=index, cos_sin_cache=build_cos_sin_cache(16, 128).to(gpu_device),
            prefix_token_count=0, rotary_dim=128, is_neox_style=True,
            source_key_buffers=src_keys, source_value_buffers=src_values,
        )


def _setup(device, *, layers=4, slots=4096, arena_slots=2048, seed=31):
    generator = torch.Generator(device=device).manual_seed(seed)
    pool = KVPool([torch.randn(slots, 4, 128, dtype=torch.bfloat16, device=device, generator=generator) for _ in range(layers)],
                  [torch.randn(slots, 4, 128, dtype=torch.bfloat16, device=device, generator=generator) for _ in range(layers)])
    arena = SnapshotArena([torch.zeros(arena_slots, 4, 128, dtype=torch.bfloat16, device=device) for _ in range(layers)],
                          [torch.zeros(arena_slots, 4, 128, dtype=torch.bfloat16, device=device) for _ in range(layers)])
    registry = LegoLinkBlockRegistry()
    executor = KVLinkExecutor(registry, RotarySpec.for_theta(4096, 128),
                              end_layer=layers, arena=arena)
    return pool, arena, registry, executor


def test_clone_blocks_survive_reuse_of_their_pool_slots(gpu_device):
    pool, arena, registry, executor = _setup(gpu_device)
    rng = np.random.default_rng(31)
    perm = rng.permutation(pool.size)
    lengths = {"clone-a": 300, "ref-b": 200, "clone-c": 150}
    slots, cursor = {}, 0
    for key, length in lengths.items():
        slots[key] = torch.from_numpy(perm[cursor : cursor + length]).to(gpu_device)
        cursor += length
        executor.capture_block(pool, key, list(range(length)), slots[key],
                               storage_mode="clone" if key.startswith("clone") else "reference")
    torch.cuda.synchronize(gpu_device)
    original_k = [bits(k) for k in pool.k_buffer]
    original_v = [bits(v) for v in pool.v_buffer]
    # The clone copies are bit-exact.
    for key in ("clone-a", "clone-c"):
        handle = registry.lookup_legolink_blocks([key]).matched_handles[0]
        for layer in range(pool.layer_num):
            assert np.array_equal(bits(arena.k_buffer[layer])[handle.kv_slots.cpu().numpy()],
                                  original_k[layer][slots[key].cpu().numpy()])
    # Reuse the clone blocks' pool slots for something else.
    for buffer in pool.k_buffer + pool.v_buffer:
        buffer.index_fill_(0, torch.cat([slots["clone-a"], slots["clone-c"]]), 0)
    plan = {"cache_keys": ["clone-c", "ref-b", "clone-a"], "recompute_initial_tokens": 8}
    resolve_link_plan(registry.get_legolink_block_tokens, [7, 8], plan)
    destination = torch.from_numpy(perm[cursor : cursor + plan["total_token_count"]]).to(gpu_device)
    prepared = executor.prepare_link(pool, destination, plan, boundary_repair_aware=True)
    prepared.launch()
    torch.cuda.synchronize(gpu_device)
    assert len(prepared.launch_info) == 2  # one launch from the arena, one from the pool
    maps = prepared.maps
    original_src = torch.cat([slots[key] for key in plan["cache_keys"]]).cpu().numpy()
    mask = np.zeros(maps.token_count, dtype=np.uint8)
    mask[prepared.repair_offsets] = 1
    expected_k, expected_v = ko.link_pool(
        original_k, original_v, original_src, maps.destination_slots.cpu().numpy(),
        maps.local_positions, maps.global_positions, build_cos_sin_cache(4096, 128).numpy(),
        key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=128, neox=True,
        prefix=maps.prefix_token_count, repair_mask=mask, rounding=ko.EAGER,
    )
    # The reference links clone blocks on its torch path (pic_runtime.py:5033-5035).
    assert prepared.rounding == "eager"
    written = maps.destination_slots.cpu().numpy()[mask == 0]
    for layer in range(pool.layer_num):
        assert np.array_equal(bits(pool.k_buffer[layer])[written], expected_k[layer][written])
        assert np.array_equal(bits(pool.v_buffer[layer])[written], expected_v[layer][written])
    # Releasing a clone block frees its arena range.
    free_before = arena.free_slots
    assert executor.release_block("clone-a")
    assert arena.free_slots == free_before + 300


def test_group_promotion_round_trip(gpu_device):
    """Link two blocks behind a prefix, promote the second block's range back
    to positions 0..n-1, then link the promoted block elsewhere."""

    pool, _, registry, executor = _setup(gpu_device, seed=41)
    rng = np.random.default_rng(41)
    theta, n_a, n_b = 1e6, 400, 250
    raw_b = rng.standard_normal((n_b, 4, 128))
    compiled_b = rope_math.rotate(raw_b, np.arange(n_b), 128, theta=theta)
    perm = rng.permutation(pool.size)
    slots_a = torch.from_numpy(perm[:n_a]).to(gpu_device)
    slots_b = torch.from_numpy(perm[n_a : n_a + n_b]).to(gpu_device)
    for layer in range(pool.layer_num):
        pool.k_buffer[layer][slots_b] = torch.from_numpy(
            ko.f32_to_bf16_bits(compiled_b.astype(np.float32)).view(np.int16)).view(torch.bfloat16).to(gpu_device)
    executor.capture_block(pool, "a", list(range(n_a)), slots_a)
    executor.capture_block(pool, "b", list(range(100, 100 + n_b)), slots_b)
    plan = {"cache_keys": ["a", "b"], "recompute_initial_tokens": 0, "physical_prefix_token_count": 3}
    resolve_link_plan(registry.get_legolink_block_tokens, [1, 2, 3, 9], plan)
    cursor = n_a + n_b
    destination = torch.from_numpy(perm[cursor : cursor + plan["total_token_count"]]).to(gpu_device)
    cursor += plan["total_token_count"]
    executor.copy_linked_kv(pool, destination, plan)
    group = plan["block_ranges"][1]
    new_slots = torch.from_numpy(perm[cursor : cursor + n_b]).to(gpu_device)
    cursor += n_b
    torch.cuda.synchronize(gpu_device)
    linked = [bits(k)[destination[group["start_token"]:group["end_token"]].cpu().numpy()] for k in pool.k_buffer]
    executor.promote_group(pool, destination, group_start=group["start_token"], group_end=group["end_token"],
                           new_slots=new_slots, cache_key="b-promoted", token_ids=list(range(100, 100 + n_b)))
    torch.cuda.synchronize(gpu_device)
    table = build_cos_sin_cache(4096, 128).numpy()
    for layer in range(pool.layer_num):
        # _promote_reconstructed_group remaps with _remap_key_positions
        # (pic_runtime.py:5914-5919): the torch path's rounding.
        expected = ko.rerotate_rows_c(linked[layer], np.arange(group["start_token"], group["end_token"]),
                                      np.arange(n_b), table, key_dtype=ko.BF16, cache_dtype=ko.F32,
                                      rotary_dim=128, neox=True, prefix=0, rounding=ko.EAGER)
        assert np.array_equal(bits(pool.k_buffer[layer])[new_slots.cpu().numpy()], expected)
    promoted = pool.k_buffer[0][new_slots].float().cpu().numpy()
    assert np.abs(promoted - compiled_b).max() < 0.06  # two bf16 re-rotations away from the original
    handle = registry.lookup_legolink_blocks(["b-promoted"]).matched_handles[0]
    assert handle.compile_local_positions == tuple(range(n_b))


def test_batched_capture_matches_block_by_block_capture(gpu_device):
    """capture_blocks copies every clone block with one launch; the arena rows,
    the handles and a link over them match what capture_block gives."""

    pool, arena, registry, executor = _setup(gpu_device, seed=53)
    rng = np.random.default_rng(53)
    perm = rng.permutation(pool.size)
    lengths = {"x-clone": 260, "y-ref": 130, "z-clone": 90, "w-clone": 1}
    blocks, cursor = [], 0
    for key, length in lengths.items():
        blocks.append({"cache_key": key, "token_ids": list(range(5, 5 + length)),
                       "slots": torch.from_numpy(perm[cursor : cursor + length]).to(gpu_device),
                       "storage_mode": "clone" if key.endswith("clone") else "reference",
                       "compile_local_positions": list(range(3, 3 + length))})
        cursor += length
    report("batched capture of three clone blocks and one reference block")
    handles = executor.capture_blocks(pool, blocks)
    torch.cuda.synchronize(gpu_device)
    assert [handle.cache_key for handle in handles] == list(lengths)
    assert arena.free_slots == arena.size - (260 + 90 + 1)
    original_k = [bits(k) for k in pool.k_buffer]
    original_v = [bits(v) for v in pool.v_buffer]
    for block, handle in zip(blocks, handles):
        assert handle.storage_mode == block["storage_mode"]
        assert handle.compile_local_positions == tuple(block["compile_local_positions"])
        source = block["slots"].cpu().numpy()
        if block["storage_mode"] == "reference":
            assert np.array_equal(handle.kv_slots.cpu().numpy(), source)
            continue
        held = handle.kv_slots.cpu().numpy()
        for layer in range(pool.layer_num):
            assert np.array_equal(bits(arena.k_buffer[layer])[held], original_k[layer][source])
            assert np.array_equal(bits(arena.v_buffer[layer])[held], original_v[layer][source])

    # An arena too small for the batch leaves no block registered and no range taken.
    free_before = arena.free_slots
    too_big = [{"cache_key": "fits", "token_ids": [1] * 8, "slots": blocks[0]["slots"][:8], "storage_mode": "clone"},
               {"cache_key": "overflow", "token_ids": [1] * (free_before + 1),
                "slots": torch.arange(free_before + 1, device=gpu_device), "storage_mode": "clone"}]
    with pytest.raises(Exception, match="free slots"):
        executor.capture_blocks(pool, too_big)
    assert arena.free_slots == free_before
    assert registry.lookup_legolink_blocks(["fits"]).matched_handles == []

    # Link the batch-captured blocks after their pool slots were reused.
    clone_slots = torch.cat([block["slots"] for block in blocks if block["storage_mode"] == "clone"])
    for buffer in pool.k_buffer + pool.v_buffer:
        buffer.index_fill_(0, clone_slots, 0)
    plan = {"cache_keys": ["z-clone", "y-ref", "x-clone", "w-clone"], "recompute_initial_tokens": 4}
    resolve_link_plan(registry.get_legolink_block_tokens, [7, 8, 9], plan)
    destination = torch.from_numpy(perm[cursor : cursor + plan["total_token_count"]]).to(gpu_device)
    prepared = executor.prepare_link(pool, destination, plan, boundary_repair_aware=True)
    prepared.launch()
    torch.cuda.synchronize(gpu_device)
    maps = prepared.maps
    by_key = {block["cache_key"]: block["slots"] for block in blocks}
    original_src = torch.cat([by_key[key] for key in plan["cache_keys"]]).cpu().numpy()
    mask = np.zeros(maps.token_count, dtype=np.uint8)
    mask[prepared.repair_offsets] = 1
    expected_k, expected_v = ko.link_pool(
        original_k, original_v, original_src, maps.destination_slots.cpu().numpy(),
        maps.local_positions, maps.global_positions, build_cos_sin_cache(4096, 128).numpy(),
        key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=128, neox=True,
        prefix=maps.prefix_token_count, repair_mask=mask, rounding=ko.EAGER,
    )
    # The reference links clone blocks on its torch path (pic_runtime.py:5033-5035).
    assert prepared.rounding == "eager"
    written = maps.destination_slots.cpu().numpy()[mask == 0]
    for layer in range(pool.layer_num):
        assert np.array_equal(bits(pool.k_buffer[layer])[written], expected_k[layer][written])
        assert np.array_equal(bits(pool.v_buffer[layer])[written], expected_v[layer][written])
