"""GPU tests of the link executor (registry -> plan -> HIP link -> repair write)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from legolink_amd import kv_link
from legolink_amd.link_plan import resolve_link_plan
from legolink_amd.link_runtime import KVLinkExecutor, KVPool, LinkRuntimeError
from legolink_amd.registry import LegoLinkBlockRegistry
from legolink_amd.rope import RotarySpec
from oracle import kv_link_oracle as ko
from tests import rope_math
from tests.gpu_helpers import bits, report

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def _bf16(array: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(ko.f32_to_bf16_bits(array.astype(np.float32)).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("case", GOLDEN["first_block_remap"]["cases"], ids=lambda c: str(c["blocks"]))
def test_first_block_remap_cases(gpu_device, case):
    """tests/pic/test_first_block_rope_remap.py:126-249 through the HIP executor:
    every block lands rotated to its request-global positions; a block already
    at its compile positions is copied bit for bit."""

    report(f"first-block case {case['blocks']}")
    heads = GOLDEN["first_block_remap"]["heads"]
    rotary = GOLDEN["first_block_remap"]["rotary_dim"]
    theta = GOLDEN["first_block_remap"]["theta"]
    rng = np.random.default_rng(20260824)
    registry = LegoLinkBlockRegistry()
    pool = KVPool.allocate(num_slots=256, num_layers=1, num_heads=heads, head_dim=rotary, device=gpu_device)
    pool.k_buffer[0].zero_()
    pool.v_buffer[0].zero_()
    raws, slot = {}, 128
    for index, (_, count) in enumerate(case["blocks"]):
        key = f"block-{index}"
        raw = rng.standard_normal((count, heads, rotary))
        compiled = rope_math.rotate(raw, np.arange(count), rotary, theta=theta)
        slots = torch.arange(slot, slot + count)
        pool.k_buffer[0][slots] = _bf16(compiled).to(gpu_device)
        pool.v_buffer[0][slots] = _bf16(rng.standard_normal((count, heads, rotary))).to(gpu_device)
        registry.register_legolink_block(key, list(range(count)), slots.to(gpu_device))
        raws[key] = (raw, compiled)
        slot += count
    total = max(start + count for start, count in case["blocks"])
    destination = torch.arange(total, device=gpu_device)
    plan = {"cache_keys": list(raws),
            "block_ranges": [{"start_token": s, "end_token": s + c} for s, c in case["blocks"]]}
    rotary_spec = RotarySpec.for_theta(4096, rotary, theta=theta)
    executor = KVLinkExecutor(registry, rotary_spec, end_layer=1)
    record = executor.copy_linked_kv(pool, destination, plan)
    torch.cuda.synchronize(gpu_device)
    assert record["rope_remapped"] == case["expected_remapped"]
    for index, (start, count) in enumerate(case["blocks"]):
        raw, compiled = raws[f"block-{index}"]
        got = pool.k_buffer[0][start : start + count].float().cpu().numpy()
        want = rope_math.rotate(raw, start + np.arange(count), rotary, theta=theta)
        assert np.abs(got - want).max() < 0.05
        if not case["expected_remapped"][index]:
            assert np.array_equal(bits(pool.k_buffer[0][start : start + count]),
                                  ko.f32_to_bf16_bits(compiled.astype(np.float32)))


def _flow(device, *, boundary_repair_aware, compact, seed=3, fused_mode="required", visit_order=None):
    """Register 5 blocks, derive a plan, link, write repaired rows; the result is
    checked with the oracle of the rounding the fused mode selects."""

    rng = np.random.default_rng(seed)
    layers, heads, dim, slots = 6, 4, 128, 8192
    lengths = [300, 77, 512, 129, 64]
    registry = LegoLinkBlockRegistry()
    generator = torch.Generator(device=device).manual_seed(seed)
    pool = KVPool([torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=device, generator=generator)
                   for _ in range(layers)],
                  [torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=device, generator=generator)
                   for _ in range(layers)])
    perm = rng.permutation(slots)
    cursor = 0
    blocks = {}
    for index, length in enumerate(lengths):
        key = f"blk{index}"
        tokens = rng.integers(0, 50_000, size=length).tolist()
        # Block 3 was compiled behind a 900-token prefix.
        positions = (np.arange(length) + 900).tolist() if index == 3 else None
        registry.register_legolink_block(key, tokens, torch.from_numpy(perm[cursor : cursor + length]).to(device),
                                         compile_local_positions=positions)
        blocks[key] = tokens
        cursor += length
    plan = {"cache_keys": ["blk2", "blk0", "blk4", "blk3", "blk1"], "recompute_initial_tokens": 16,
            "physical_prefix_token_count": 5}
    host_tokens = rng.integers(0, 50_000, size=5 + 40).tolist()
    linked = resolve_link_plan(registry.get_legolink_block_tokens, host_tokens, plan)
    destination = torch.from_numpy(perm[cursor : cursor + len(linked)]).to(device)
    rotary = RotarySpec.for_theta(2048, dim)
    executor = KVLinkExecutor(registry, rotary, end_layer=layers, fused_mode=fused_mode, visit_order=visit_order)
    before_k = [bits(k) for k in pool.k_buffer]
    before_v = [bits(v) for v in pool.v_buffer]
    prepared = executor.prepare_link(pool, destination, plan, boundary_repair_aware=boundary_repair_aware,
                                     compact_repair_rows=compact)
    prepared.launch()
    repair_rows = int(prepared.repair_offsets.size)
    repaired_k = torch.randn(layers, repair_rows, heads, dim, dtype=torch.bfloat16, device=device, generator=generator)
    repaired_v = torch.randn_like(repaired_k)
    if repair_rows:
        prepared.write_repaired(repaired_k, repaired_v)
    torch.cuda.synchronize(device)
    maps = prepared.maps
    mask = np.zeros(maps.token_count, dtype=np.uint8)
    mask[prepared.repair_offsets] = 1
    expected_k, expected_v = ko.link_pool(
        before_k, before_v, maps.source_slots.cpu().numpy(), maps.destination_slots.cpu().numpy(),
        maps.local_positions, maps.global_positions, rotary.cos_sin_cache.cpu().numpy(),
        key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=dim, neox=True,
        prefix=maps.prefix_token_count, repair_mask=mask if repair_rows else None,
        rounding=ko.EAGER if prepared.rounding == "eager" else ko.FUSED,
    )
    if repair_rows:
        expected_k, expected_v = ko.scatter_rows(expected_k, expected_v,
                                                 prepared.repair_destination_slots.cpu().numpy(),
                                                 bits(repaired_k), bits(repaired_v))
    for layer in range(layers):
        assert np.array_equal(bits(pool.k_buffer[layer]), expected_k[layer]), f"K layer {layer}"
        assert np.array_equal(bits(pool.v_buffer[layer]), expected_v[layer]), f"V layer {layer}"
    return prepared, [bits(k) for k in pool.k_buffer], plan


@pytest.mark.parametrize("visit_order", ["plan", "source", "destination"])
@pytest.mark.parametrize("compact", [True, False])
def test_visit_orders_match_oracle(gpu_device, visit_order, compact):
    """The order in which the kernel visits the rotated rows changes nothing:
    every order, with repair rows compacted or masked, equals the oracle."""

    report(f"visit order {visit_order}, compact {compact}")
    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=True, compact=compact, visit_order=visit_order)
    assert prepared.visit_order == visit_order


def test_single_request_visits_destination_order(gpu_device):
    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=True, compact=True)
    assert prepared.visit_order == "destination"
    maps = prepared._kernel_maps[0]
    prefix = prepared.segment_plan.set_prefix[0]
    destinations = maps[1, prefix:].cpu().numpy()
    assert np.all(np.diff(destinations) > 0)


def test_plan_link_repair_flow_matches_oracle(gpu_device):
    prepared, _, plan = _flow(gpu_device, boundary_repair_aware=True, compact=True)
    # imp_indices inside blocks: 16 per block after the first (4 seams).
    assert prepared.repair_offsets.size == 4 * 16
    assert prepared.maps.block_specs[3]["needs_rope_remap"]
    assert prepared.linked_token_count == prepared.maps.token_count - 64


@pytest.mark.parametrize("fused_mode,rounding", [("disabled", "eager"), ("auto", "fused"), ("1", "fused")])
def test_fused_mode_selects_the_rounding(gpu_device, fused_mode, rounding):
    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=True, compact=True, seed=21, fused_mode=fused_mode)
    assert prepared.rounding == rounding
    assert prepared.record()["rounding"] == rounding


def test_fused_mode_defaults_to_the_environment(gpu_device, monkeypatch):
    monkeypatch.delenv("SGLANG_PIC_TRITON_FUSED_KV_LINK", raising=False)
    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=True, compact=True, seed=22, fused_mode=None)
    assert prepared.rounding == "eager"  # the reference's default: its torch path
    monkeypatch.setenv("SGLANG_PIC_TRITON_FUSED_KV_LINK", "required")
    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=True, compact=True, seed=22, fused_mode=None)
    assert prepared.rounding == "fused"


def test_compacted_and_masked_links_agree(gpu_device):
    _, compacted, _ = _flow(gpu_device, boundary_repair_aware=True, compact=True, seed=9)
    _, masked, _ = _flow(gpu_device, boundary_repair_aware=True, compact=False, seed=9)
    for a, b in zip(compacted, masked):
        assert np.array_equal(a, b)


def test_link_without_repair_awareness_copies_every_token(gpu_device):
    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=False, compact=True, seed=5)
    assert prepared.repair_offsets.size == 0
    assert prepared.linked_token_count == prepared.maps.token_count


def test_executor_matches_the_per_layer_drop_in_operator(gpu_device):
    layers, slots = 4, 4096
    rng = np.random.default_rng(12)
    registry = LegoLinkBlockRegistry()
    generator = torch.Generator(device=gpu_device).manual_seed(12)
    keys = [torch.randn(slots, 4, 128, dtype=torch.bfloat16, device=gpu_device, generator=generator) for _ in range(layers)]
    values = [torch.randn(slots, 4, 128, dtype=torch.bfloat16, device=gpu_device, generator=generator) for _ in range(layers)]
    keys_b, values_b = [k.clone() for k in keys], [v.clone() for v in values]
    perm = rng.permutation(slots)
    registry.register_legolink_block("x", list(range(700)), torch.from_numpy(perm[:700]).to(gpu_device))
    registry.register_legolink_block("y", list(range(300)), torch.from_numpy(perm[700:1000]).to(gpu_device))
    plan = {"cache_keys": ["y", "x"], "block_ranges": [{"start_token": 0, "end_token": 300},
                                                     {"start_token": 300, "end_token": 1000}]}
    destination = torch.from_numpy(perm[1000:2000]).to(gpu_device)
    rotary = RotarySpec.for_theta(2048, 128)
    executor = KVLinkExecutor(registry, rotary, end_layer=layers, fused_mode="required")
    executor.copy_linked_kv(KVPool(keys, values), destination, plan)
    maps = executor.build_link_maps(destination, plan)
    local = torch.from_numpy(maps.local_positions).to(gpu_device)
    glob = torch.from_numpy(maps.global_positions).to(gpu_device)
    for key, value in zip(keys_b, values_b):
        kv_link.fused_kv_link_inplace(
            key_buffer=key, value_buffer=value, source_slots=maps.source_slots,
            destination_slots=maps.destination_slots, local_positions=local, global_positions=glob,
            cos_sin_cache=rotary.cos_sin_cache, prefix_token_count=maps.prefix_token_count,
            rotary_dim=128, is_neox_style=True,
        )
    torch.cuda.synchronize(gpu_device)
    assert maps.prefix_token_count == 300  # block "y" sits at its compile positions
    for a, b in zip(keys + values, keys_b + values_b):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_prepared_link_replays_in_a_hip_graph(gpu_device):
    """The link and the repair write allocate nothing and sync nothing, so they
    can be captured; every replay must equal the eager result."""

    layers, slots, heads, dim = 3, 2048, 4, 128
    rng = np.random.default_rng(4)
    registry = LegoLinkBlockRegistry()
    generator = torch.Generator(device=gpu_device).manual_seed(4)
    pool = KVPool([torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator) for _ in range(layers)],
                  [torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator) for _ in range(layers)])
    perm = rng.permutation(slots)
    registry.register_legolink_block("a", list(range(400)), torch.from_numpy(perm[:400]).to(gpu_device))
    registry.register_legolink_block("b", list(range(250)), torch.from_numpy(perm[400:650]).to(gpu_device))
    plan = {"cache_keys": ["a", "b"], "recompute_initial_tokens": 8}
    resolve_link_plan(registry.get_legolink_block_tokens, [1, 2, 3], plan)
    destination = torch.from_numpy(perm[650:1400]).to(gpu_device)
    executor = KVLinkExecutor(registry, RotarySpec.for_theta(1024, dim), end_layer=layers)
    prepared = executor.prepare_link(pool, destination, plan, boundary_repair_aware=True)
    repaired_k = torch.randn(layers, int(prepared.repair_offsets.size), heads, dim, dtype=torch.bfloat16,
                             device=gpu_device, generator=generator)
    repaired_v = torch.randn_like(repaired_k)
    write = prepared.prepare_write_repaired(repaired_k, repaired_v)
    touched = prepared.maps.destination_slots
    prepared.launch()
    write()
    torch.cuda.synchronize(gpu_device)
    expected = [bits(k) for k in pool.k_buffer] + [bits(v) for v in pool.v_buffer]

    stream = torch.cuda.Stream(device=gpu_device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            prepared.launch()
            write()
    torch.cuda.synchronize(gpu_device)
    for replay in range(3):
        for buffer in pool.k_buffer + pool.v_buffer:
            buffer.index_fill_(0, touched, 0)  # eager work between replays
        torch.cuda.synchronize(gpu_device)
        graph.replay()
        torch.cuda.synchronize(gpu_device)
        actual = [bits(k) for k in pool.k_buffer] + [bits(v) for v in pool.v_buffer]
        for a, b in zip(actual, expected):
            assert np.array_equal(a, b), f"replay {replay}"


@pytest.mark.parametrize("mix", ["clone_in_every_request", "mixed"])
@pytest.mark.parametrize("fused_mode", ["disabled", "auto"])
@pytest.mark.parametrize("order_by_source", [True, False])
def test_batched_link_equals_request_by_request_links(gpu_device, order_by_source, fused_mode, mix):
    """prepare_links over several requests -- identity first blocks, a request
    behind a chat prefix, a block compiled behind a prefix, clone blocks in
    the snapshot arena, shared blocks, repair rows -- leaves the pool
    bit-identical to linking and repairing each request alone, whether the
    kernel visits the rows in plan order or in source-slot order.  With
    "mixed", some requests hold no clone block: under "auto" those link with
    the fused rounding and the others with the eager one, each as its own
    link would (pic_runtime.py:5033-5035 decides per request)."""

    from legolink_amd.link_runtime import SnapshotArena

    layers, slots, heads, dim = 3, 8192, 4, 128
    rng = np.random.default_rng(31)
    generator = torch.Generator(device=gpu_device).manual_seed(31)
    keys = [torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator)
            for _ in range(layers)]
    values = [torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator)
              for _ in range(layers)]
    pool_a = KVPool(keys, values)
    pool_b = KVPool([k.clone() for k in keys], [v.clone() for v in values])
    arena = SnapshotArena.allocate(num_slots=2048, num_layers=layers, num_heads=heads, head_dim=dim,
                                   device=gpu_device)
    registry = LegoLinkBlockRegistry()
    rotary = RotarySpec.for_theta(8192, dim)
    executor = KVLinkExecutor(registry, rotary, end_layer=layers, arena=arena, fused_mode=fused_mode)
    perm = rng.permutation(slots)
    cursor = 0
    lengths = [120, 64, 300, 45, 200, 90]
    for index, length in enumerate(lengths):
        block_slots = torch.from_numpy(perm[cursor : cursor + length]).to(gpu_device)
        cursor += length
        positions = (np.arange(length) + 700).tolist() if index == 3 else None
        executor.capture_block(pool_a, f"b{index}", list(range(length)), block_slots,
                               storage_mode="clone" if index in (1, 4) else "reference",
                               compile_local_positions=positions)
    torch.cuda.synchronize(gpu_device)

    def plan_of(names, start=0):
        ranges, cursor_ = [], start
        for name in names:
            count = lengths[int(name[1:])]
            ranges.append({"start_token": cursor_, "end_token": cursor_ + count})
            cursor_ += count
        imp = [r["start_token"] + k for r in ranges[1:] for k in range(8)]
        return {"cache_keys": list(names), "block_ranges": ranges, "imp_indices": imp}, cursor_

    requests = []
    request_names = [(["b0", "b1", "b2"], 0), (["b4", "b3"], 5), (["b1", "b5", "b0"], 0), (["b2", "b4"], 0)]
    if mix == "mixed":  # requests of reference blocks only, around and between the others
        request_names = ([(["b3", "b0"], 0)] + request_names[:2] + [(["b5", "b2", "b3"], 7)]
                         + request_names[2:] + [(["b0", "b5"], 0)])
    for names, start in request_names:
        plan, total = plan_of(names, start)
        destination = torch.from_numpy(perm[cursor : cursor + total]).to(gpu_device)
        cursor += total
        requests.append((destination, plan))
    report(f"batched link: {len(requests)} requests, {cursor} slots used")

    batched = executor.prepare_links(pool_a, requests, boundary_repair_aware=True, order_by_source=order_by_source)
    assert batched.order_by_source == order_by_source
    holds_clone = [any(name in ("b1", "b4") for name in names) for names, _ in request_names]
    want_roundings = ["eager" if fused_mode == "disabled" or clone else "fused" for clone in holds_clone]
    assert batched.request_roundings == want_roundings
    # A request holding a clone block takes the reference's torch path; under
    # "auto" the other requests keep the fused kernel's rounding.
    assert batched.rounding == ("mixed" if len(set(want_roundings)) > 1 else "eager")
    assert batched.fallback_reason == (None if fused_mode == "disabled" else "reference_storage_required")
    batched.launch()
    rows = int(batched.repair_offsets.size)
    repaired_k = torch.randn(layers, rows, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator)
    repaired_v = torch.randn_like(repaired_k)
    batched.write_repaired(repaired_k, repaired_v)
    # One launch per source (pool, arena); a mixed pool set splits into a
    # fused and an eager launch.
    assert len(batched.launch_info) == (3 if batched.rounding == "mixed" else 2)

    row = 0
    for (destination, plan), rounding in zip(requests, want_roundings):
        single = executor.prepare_link(pool_b, destination, plan, boundary_repair_aware=True)
        assert single.rounding == rounding
        single.launch()
        count = int(single.repair_offsets.size)
        single.write_repaired(repaired_k[:, row : row + count].contiguous(),
                              repaired_v[:, row : row + count].contiguous())
        row += count
    assert row == rows
    torch.cuda.synchronize(gpu_device)
    for a, b in zip(pool_a.k_buffer + pool_a.v_buffer, pool_b.k_buffer + pool_b.v_buffer):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_streamed_single_request_link_matches_oracle(gpu_device, monkeypatch):
    """With the memory-side-cache threshold lowered to 0 a single request's link
    takes the non-temporal row loads; it still matches the oracle bit for bit
    (the flow helper checks every layer), and small links keep cached loads."""

    from legolink_amd import link_runtime

    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=True, compact=True, seed=13)
    assert not prepared.stream_source_rows  # a few MB: may be cache-resident
    monkeypatch.setattr(link_runtime, "MEMORY_SIDE_CACHE_BYTES", 0)
    prepared, _, _ = _flow(gpu_device, boundary_repair_aware=True, compact=True, seed=13)
    assert prepared.stream_source_rows
    assert all(info["kernel"] == "vector" for info in prepared.launch_info)


def test_required_fused_mode_refuses_clone_blocks(gpu_device):
    """pic_runtime.py:5033-5035, :5153-5157: the fused kernel needs every block in
    pool slots; "required" fails with the reference's message."""

    from legolink_amd.errors import LinkRuntimeError
    from legolink_amd.link_runtime import SnapshotArena

    layers, slots = 2, 1024
    pool = KVPool.allocate(num_slots=slots, num_layers=layers, num_heads=4, head_dim=128, device=gpu_device)
    arena = SnapshotArena.allocate(num_slots=256, num_layers=layers, num_heads=4, head_dim=128, device=gpu_device)
    registry = LegoLinkBlockRegistry()
    executor = KVLinkExecutor(registry, RotarySpec.for_theta(1024, 128),
                              end_layer=layers, arena=arena, fused_mode="required")
    executor.capture_block(pool, "c", list(range(50)), torch.arange(50, device=gpu_device), storage_mode="clone")
    plan = {"cache_keys": ["c"], "block_ranges": [{"start_token": 10, "end_token": 60}]}
    with pytest.raises(LinkRuntimeError, match="Required Triton LegoLink fusion is unavailable: "
                                               "reference_storage_required"):
        executor.prepare_link(pool, torch.arange(100, 200, device=gpu_device), plan)


def test_executor_counts_tokens_skipped_for_bad_slots(gpu_device):
    """A block registered with slots outside the pool: the kernel skips those
    tokens, the executor's device counter holds how many, and
    check_skipped_rows raises once (then the count starts again at zero)."""

    report("executor skipped-row counter: 2 blocks, 5 bad slots")
    layers, slots, heads, dim = 3, 1500, 4, 128
    rng = np.random.default_rng(8)
    registry = LegoLinkBlockRegistry()
    generator = torch.Generator(device=gpu_device).manual_seed(9)
    pool = KVPool([torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator) for _ in range(layers)],
                  [torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator) for _ in range(layers)])
    perm = rng.permutation(slots)
    bad = perm[:300].copy()
    bad[[3, 50, 51, 200, 299]] = slots + np.array([0, 1, 7, 100, 5])
    registry.register_legolink_block("a", list(range(400)), torch.from_numpy(perm[300:700]).to(gpu_device))
    registry.register_legolink_block("b", list(range(300)), torch.from_numpy(bad).to(gpu_device))
    plan = {"cache_keys": ["a", "b"], "recompute_initial_tokens": 8}
    resolve_link_plan(registry.get_legolink_block_tokens, [1, 2, 3], plan)
    destination = torch.from_numpy(perm[700:1400]).to(gpu_device)
    executor = KVLinkExecutor(registry, RotarySpec.for_theta(1024, dim), end_layer=layers)
    before = [bits(k) for k in pool.k_buffer]
    executor.prepare_link(pool, destination, plan, boundary_repair_aware=False).launch()
    with pytest.raises(LinkRuntimeError, match="skipped 5 token"):
        executor.check_skipped_rows()
    executor.check_skipped_rows()  # reset by the failed check
    # The skipped tokens' destinations (block b starts at request position 400) were not written.
    untouched = destination.cpu().numpy()[400 + np.array([3, 50, 51, 200, 299])]
    for layer in range(layers):
        assert np.array_equal(bits(pool.k_buffer[layer])[untouched], before[layer][untouched])
    # A clean link leaves the counter at zero.
    registry.register_legolink_block("c", list(range(300)), torch.from_numpy(perm[:300]).to(gpu_device))
    plan = {"cache_keys": ["a", "c"], "recompute_initial_tokens": 8}
    resolve_link_plan(registry.get_legolink_block_tokens, [1, 2, 3], plan)
    executor.prepare_link(pool, destination, plan, boundary_repair_aware=False).launch()
    assert executor.skipped_rows() == 0


class _ScaledRotary:
    """A model rotary module with linear position scaling (row p holds the
    angles of p / scale): its table grows through its own method, as sglang's
    rotary embeddings do."""

    def __init__(self, rows, rotary_dim, theta, scale, device):
        self.rotary_dim, self.is_neox_style = rotary_dim, True
        self.theta, self.scale, self.device, self.grown_to = theta, scale, device, []
        self.cos_sin_cache = self._table(rows)

    def _table(self, rows):
        inv_freq = 1.0 / self.theta ** (torch.arange(0, self.rotary_dim, 2, dtype=torch.float32) / self.rotary_dim)
        angles = torch.outer(torch.arange(rows, dtype=torch.float32) / self.scale, inv_freq)
        return torch.cat((angles.cos(), angles.sin()), dim=-1).to(self.device)

    def _ensure_cos_sin_cache_length(self, needed_max_pos):
        if needed_max_pos >= self.cos_sin_cache.shape[0]:
            self.grown_to.append(needed_max_pos)
            self.cos_sin_cache = self._table(needed_max_pos + 1)


def test_link_grows_a_model_rotary_table_through_the_module(gpu_device):
    """The executor given a model's rotary module: a link past the end of its
    table grows it through the module (pic_runtime.py:5051-5053), keeping the
    module's scaling, and the link is bit-exact against the oracle on the
    grown table."""

    report("rotary module growth: 2 blocks, positions up to 1099, table of 300 rows, scale 2")
    layers, heads, dim, slots = 3, 4, 128, 4096
    rng = np.random.default_rng(12)
    generator = torch.Generator(device=gpu_device).manual_seed(12)
    pool = KVPool([torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator)
                   for _ in range(layers)],
                  [torch.randn(slots, heads, dim, dtype=torch.bfloat16, device=gpu_device, generator=generator)
                   for _ in range(layers)])
    perm = rng.permutation(slots)
    registry = LegoLinkBlockRegistry()
    registry.register_legolink_block("a", list(range(200)), torch.from_numpy(perm[:200]).to(gpu_device))
    registry.register_legolink_block("b", list(range(300)), torch.from_numpy(perm[200:500]).to(gpu_device))
    destination = torch.from_numpy(perm[500:1600]).to(gpu_device)
    plan = {"cache_keys": ["a", "b"],
            "block_ranges": [{"start_token": 0, "end_token": 200}, {"start_token": 800, "end_token": 1100}]}
    module = _ScaledRotary(300, dim, 1e6, 2.0, gpu_device)
    executor = KVLinkExecutor(registry, module, end_layer=layers, fused_mode="required")
    before_k = [bits(k) for k in pool.k_buffer]
    before_v = [bits(v) for v in pool.v_buffer]
    executor.copy_linked_kv(pool, destination, plan)
    torch.cuda.synchronize(gpu_device)
    assert module.grown_to and module.cos_sin_cache.shape[0] >= 1100
    assert executor.rotary_by_layer[0].cos_sin_cache is module.cos_sin_cache
    executor.check_skipped_rows()
    src = perm[:500]
    positions = np.concatenate([np.arange(200), np.arange(800, 1100)])
    local = np.concatenate([np.arange(200), np.arange(300)])
    dst = perm[500:1600][positions]
    want_k, want_v = ko.link_pool(before_k, before_v, src, dst, local, positions,
                                  module.cos_sin_cache.cpu().numpy(), key_dtype=ko.BF16, cache_dtype=ko.F32,
                                  rotary_dim=dim, neox=True, prefix=200)
    for layer in range(layers):
        assert np.array_equal(bits(pool.k_buffer[layer]), want_k[layer]), f"K layer {layer}"
        assert np.array_equal(bits(pool.v_buffer[layer]), want_v[layer]), f"V layer {layer}"
