"""Helpers shared by the GPU parity tests: pools, bit views, oracle comparison."""

from __future__ import annotations

import sys

import numpy as np
import torch

from legolink_amd import kv_link
from legolink_amd.rope import build_cos_sin_cache
from legolink_amd.workloads import LinkWorkload
from oracle import kv_link_oracle as ko

TORCH_TO_CODE = {torch.bfloat16: ko.BF16, torch.float16: ko.F16, torch.float32: ko.F32}


def report(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def bits(tensor: torch.Tensor) -> np.ndarray:
    """uint16 bit patterns of a bf16/fp16 tensor, on the host."""

    return tensor.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def cache_host(cache: torch.Tensor) -> np.ndarray:
    if cache.dtype == torch.float32:
        return cache.detach().cpu().numpy()
    return bits(cache)


def make_pool(layers: int, slots: int, heads: int, key_dim: int, value_dim: int,
              dtype: torch.dtype, device: torch.device, seed: int) -> tuple[list, list]:
    generator = torch.Generator(device=device).manual_seed(seed)
    keys = [torch.randn(slots, heads, key_dim, dtype=dtype, device=device, generator=generator)
            for _ in range(layers)]
    values = [torch.randn(slots, heads, value_dim, dtype=dtype, device=device, generator=generator)
              for _ in range(layers)]
    return keys, values


_HASH_WEIGHTS: dict = {}


def row_checksums(buffer: torch.Tensor, chunk: int = 65536) -> torch.Tensor:
    """Per-slot hash of a row's element bit patterns (int64), on the device:
    sum_i w_i * bits_i with a distinct pseudo-random weight w_i in
    [1, 2^20] per element position, so that a stray write that swaps two
    elements of a row, or copies in a row with the same plain sum, changes
    it.  |bits| < 2^15 and at most 2^11 elements per row keep the sum below
    2^46: exact in int64."""

    elements = buffer[0].numel()
    assert elements <= 2048
    key = (buffer.device, elements)
    weights = _HASH_WEIGHTS.get(key)
    if weights is None:
        index = torch.arange(elements, dtype=torch.int64)
        weights = ((index * 2654435761) % (1 << 20) + 1).to(buffer.device)
        _HASH_WEIGHTS[key] = weights
    flat = buffer.view(torch.int16).reshape(buffer.shape[0], elements)
    parts = [(flat[i : i + chunk].to(torch.int64) * weights).sum(dim=1) for i in range(0, flat.shape[0], chunk)]
    return torch.cat(parts)


def _link_through_executor(workload: LinkWorkload, keys, values, table, repaired_k, repaired_v,
                           device, *, fused_mode: str, with_scatter: bool) -> dict:
    """The link step exactly as bench.py runs it: blocks registered, the plan
    prepared by the executor (map builder on the device, repair rows left out
    of the maps, non-temporal row loads for a single request larger than the
    memory-side cache), then the link launch and the repaired-row write-back."""

    from legolink_amd.link_runtime import KVLinkExecutor, KVPool
    from legolink_amd.registry import LegoLinkBlockRegistry
    from legolink_amd.rope import RotarySpec

    registry = LegoLinkBlockRegistry()
    blocks, requests = workload.link_requests()
    for key, (source, local) in blocks.items():
        registry.register_legolink_block(key, range(source.size), torch.from_numpy(source).to(device),
                                         compile_local_positions=local.tolist())
    executor = KVLinkExecutor(registry, RotarySpec(table, rotary_dim=workload.rotary_dim),
                              end_layer=workload.shape.layers, fused_mode=fused_mode)
    pool = KVPool(keys, values)
    requests = [(torch.from_numpy(slots).to(device), plan) for slots, plan in requests]
    if len(requests) == 1:
        prepared = executor.prepare_link(pool, requests[0][0], requests[0][1], boundary_repair_aware=True,
                                         compact_repair_rows=True)
    else:
        prepared = executor.prepare_links(pool, requests, boundary_repair_aware=True, compact_repair_rows=True)
    assert prepared.linked_token_count == workload.tokens - workload.repair_rows
    assert np.array_equal(prepared.repair_destination_slots.cpu().numpy(), workload.repair_destination_slots)
    launch = dict(prepared.launch_info[0], stream_source_rows=bool(prepared.stream_source_rows),
                  rounding=prepared.rounding, visit_order=prepared.visit_order)
    report(f"[{workload.name}] executor link {launch}")
    prepared.launch()
    if with_scatter:
        prepared.write_repaired(repaired_k, repaired_v)
    return launch


def check_workload(
    workload: LinkWorkload,
    device: torch.device,
    *,
    sample_tokens: int | None = None,
    with_scatter: bool = True,
    kernel: int = 0,
    seed: int = 7,
    rounding: str = "fused",
    via_executor: bool = False,
) -> dict:
    """Run one link step (link + repaired-row scatter) of ``workload`` on the GPU
    and compare it with the oracle.  ``via_executor`` runs it through
    KVLinkExecutor.prepare_link as bench.py does (then the fused mode follows
    ``rounding``: "required" for fused, "disabled" for eager); otherwise
    through the all-layer operator with a repair mask.  Returns summary counts."""

    shape = workload.shape
    report(f"[{workload.name}] pool {workload.num_slots} slots x {shape.layers} layers, "
           f"{workload.tokens} tokens, {workload.repair_rows} repair rows")
    keys, values = make_pool(shape.layers, workload.num_slots, shape.kv_heads, shape.head_dim,
                             shape.head_dim, torch.bfloat16, device, seed)
    table = build_cos_sin_cache(workload.max_position + 1, workload.rotary_dim,
                                theta=workload.theta).to(device)
    src = torch.from_numpy(workload.source_slots).to(device)
    dst = torch.from_numpy(workload.destination_slots).to(device)
    local = torch.from_numpy(workload.local_positions).to(device)
    glob = torch.from_numpy(workload.global_positions).to(device)
    mask = torch.from_numpy(workload.repair_mask).to(device)
    repair_offsets = torch.from_numpy(workload.repair_offsets).to(device)
    repair_slots = dst.index_select(0, repair_offsets)
    generator = torch.Generator(device=device).manual_seed(seed + 1)
    repaired_k = torch.randn(shape.layers, workload.repair_rows, shape.kv_heads, shape.head_dim,
                             dtype=torch.bfloat16, device=device, generator=generator)
    repaired_v = torch.randn_like(repaired_k)

    if sample_tokens is None or sample_tokens >= workload.tokens:
        tokens = np.arange(workload.tokens)
    else:
        rng = np.random.default_rng(seed)
        tokens = np.sort(rng.choice(workload.tokens, size=sample_tokens, replace=False))
    tok = torch.from_numpy(tokens).to(device)
    src_t, dst_t = src.index_select(0, tok), dst.index_select(0, tok)
    before = []
    for key, value in zip(keys, values):
        before.append((key.index_select(0, src_t), key.index_select(0, dst_t),
                       value.index_select(0, src_t), value.index_select(0, dst_t),
                       row_checksums(key), row_checksums(value)))
    torch.cuda.synchronize(device)

    launch = None
    if via_executor:
        launch = _link_through_executor(workload, keys, values, table, repaired_k, repaired_v, device,
                                        fused_mode="required" if rounding == "fused" else "disabled",
                                        with_scatter=with_scatter)
    else:
        report(f"[{workload.name}] link launch {kv_link.describe_link_launch(key_buffers=keys, value_buffers=values, source_slots=src, destination_slots=dst, local_positions=local, global_positions=glob, cos_sin_cache=table, prefix_token_count=workload.prefix_token_count, rotary_dim=workload.rotary_dim, is_neox_style=True, repair_mask=mask, kernel=kernel)}")
        kv_link.fused_kv_link_layers_inplace(
            key_buffers=keys, value_buffers=values, source_slots=src, destination_slots=dst,
            local_positions=local, global_positions=glob, cos_sin_cache=table,
            prefix_token_count=workload.prefix_token_count, rotary_dim=workload.rotary_dim,
            is_neox_style=True, repair_mask=mask, kernel=kernel, rounding=rounding,
        )
        if with_scatter:
            kv_link.scatter_kv_rows_inplace(
                key_buffers=keys, value_buffers=values, destination_slots=repair_slots,
                repaired_keys=repaired_k, repaired_values=repaired_v,
            )
    torch.cuda.synchronize(device)
    report(f"[{workload.name}] kernels done; comparing {len(tokens)} tokens with the oracle")

    local_t = workload.local_positions[tokens]
    global_t = workload.global_positions[tokens]
    prefix_t = int(np.count_nonzero(tokens < workload.prefix_token_count))
    masked_t = workload.repair_mask[tokens] != 0
    # Where each sampled repair token's repaired row sits in repaired_k.
    repair_index = np.full(workload.tokens, -1, dtype=np.int64)
    repair_index[workload.repair_offsets] = np.arange(workload.repair_rows)
    repair_index_t = repair_index[tokens]
    table_host = cache_host(table)
    dst_set = torch.zeros(workload.num_slots, dtype=torch.bool, device=device)
    dst_set[dst] = True
    untouched = ~dst_set
    mismatches = 0
    for layer, (key, value) in enumerate(zip(keys, values)):
        src_k, dst_k_before, src_v, dst_v_before, ck_k, ck_v = before[layer]
        expected_k = ko.rerotate_rows_c(
            bits(src_k), local_t, global_t, table_host, key_dtype=ko.BF16, cache_dtype=ko.F32,
            rotary_dim=workload.rotary_dim, neox=True, prefix=prefix_t,
            rounding=ko.EAGER if rounding == "eager" else ko.FUSED,
        )
        expected_v = bits(src_v)
        if with_scatter:
            repaired_rows = repair_index_t[masked_t]
            expected_k[masked_t] = bits(repaired_k[layer])[repaired_rows]
            expected_v[masked_t] = bits(repaired_v[layer])[repaired_rows]
        else:
            expected_k[masked_t] = bits(dst_k_before)[masked_t]
            expected_v[masked_t] = bits(dst_v_before)[masked_t]
        actual_k = bits(key.index_select(0, dst_t))
        actual_v = bits(value.index_select(0, dst_t))
        mismatches += int(np.count_nonzero(actual_k != expected_k))
        mismatches += int(np.count_nonzero(actual_v != expected_v))
        assert np.array_equal(actual_k, expected_k), f"{workload.name} layer {layer}: K differs"
        assert np.array_equal(actual_v, expected_v), f"{workload.name} layer {layer}: V differs"
        assert torch.equal(row_checksums(key)[untouched], ck_k[untouched]), (
            f"{workload.name} layer {layer}: K rows outside the destinations changed")
        assert torch.equal(row_checksums(value)[untouched], ck_v[untouched]), (
            f"{workload.name} layer {layer}: V rows outside the destinations changed")
    report(f"[{workload.name}] all {shape.layers} layers bit-exact ({rounding} rounding)")
    del keys, values, before
    torch.cuda.empty_cache()
    return {"tokens_checked": len(tokens), "mismatches": mismatches, "launch": launch}
