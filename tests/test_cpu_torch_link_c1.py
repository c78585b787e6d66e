"""The CPU torch link that workload c1 names, and that bench.py's cpu_baseline
times, against the oracle, bit for bit, at c1's full size.

c1: Qwen2.5-7B KV shape (28 layers x 4 KV heads x 128 dims, bf16), a pool of
65,536 slots, 4 registered blocks of 512 tokens linked in a permuted order
into one 2,048-token request, per-block position deltas in [-1536, 1536],
neox RoPE with theta 1e6, 8 imp_indices per seam.

The torch side is ``oracle/r1_torch`` -- the reference's eager batched path,
per layer index_select -> _remap_key_positions -> index_copy_
(patched_sglang_files/python/sglang/srt/pic_runtime.py:5534-5599, :6025-6058,
:1868-1885), then the repair write-back (flashinfer_sparse_repair.py:2235-2239).
The oracle side is ``kv_link_oracle.link_pool(rounding=EAGER)`` (plain C, one
rounding per operation in the cache's and then the key's dtype) followed by
``scatter_rows``.  The eager path copies the repair rows too and the
write-back then overwrites them, so the oracle link runs without a mask.
"""

from __future__ import annotations

import numpy as np
import torch

from legolink_amd.rope import build_cos_sin_cache
from legolink_amd.workloads import make_workload
from oracle import kv_link_oracle as ko
from oracle import r1_torch


def _bits(tensor: torch.Tensor) -> np.ndarray:
    return tensor.view(torch.int16).numpy().view(np.uint16)


def test_torch_link_of_c1_equals_the_eager_oracle():
    workload = make_workload("c1")
    shape = workload.shape
    slots, layers = workload.num_slots, shape.layers
    assert (slots, layers, shape.kv_heads, shape.head_dim) == (65_536, 28, 4, 128)
    assert workload.tokens == 2048 and workload.repair_rows == 24
    generator = torch.Generator().manual_seed(20260824)
    # The pool: a tiled random block (cheap to fill), then fresh N(0,1) values in
    # every row the link reads, so that no two source rows are alike.
    tile = torch.randn(1 << 20, generator=generator).to(torch.bfloat16)
    row = shape.kv_heads * shape.head_dim
    src = torch.from_numpy(workload.source_slots)
    dst = torch.from_numpy(workload.destination_slots)
    assert np.intersect1d(workload.source_slots, workload.destination_slots).size == 0

    def layer_buffer() -> torch.Tensor:
        flat = tile.repeat(slots * row // tile.numel())
        buffer = flat.view(slots, shape.kv_heads, shape.head_dim).clone()
        buffer[src] = torch.randn(workload.tokens, shape.kv_heads, shape.head_dim,
                                  generator=generator).to(torch.bfloat16)
        return buffer

    keys = [layer_buffer() for _ in range(layers)]
    values = [layer_buffer() for _ in range(layers)]
    table = build_cos_sin_cache(workload.max_position + 1, workload.rotary_dim, theta=workload.theta)
    repair_slots = workload.repair_destination_slots
    repaired_k = torch.randn(layers, workload.repair_rows, shape.kv_heads, shape.head_dim,
                             generator=generator).to(torch.bfloat16)
    repaired_v = torch.randn(layers, workload.repair_rows, shape.kv_heads, shape.head_dim,
                             generator=generator).to(torch.bfloat16)

    # Expected rows, layer by layer, from the pool before the torch link runs:
    # only the destination rows change, so only they are kept.
    expected_k, expected_v = [], []
    for layer in range(layers):
        link_k, link_v = ko.link_pool(
            [_bits(keys[layer])], [_bits(values[layer])], workload.source_slots, workload.destination_slots,
            workload.local_positions, workload.global_positions, table.numpy(), key_dtype=ko.BF16,
            cache_dtype=ko.F32, rotary_dim=workload.rotary_dim, neox=True, prefix=workload.prefix_token_count,
            rounding=ko.EAGER)
        link_k, link_v = ko.scatter_rows(link_k, link_v, repair_slots, _bits(repaired_k[layer : layer + 1]),
                                         _bits(repaired_v[layer : layer + 1]))
        expected_k.append(link_k[0][workload.destination_slots])
        expected_v.append(link_v[0][workload.destination_slots])
        del link_k, link_v
    untouched = np.setdiff1d(np.arange(slots), workload.destination_slots)[::97]
    before_k = [_bits(k)[untouched].copy() for k in keys]
    before_v = [_bits(v)[untouched].copy() for v in values]

    r1_torch.link_batched_layers(keys, values, src, dst, torch.from_numpy(workload.local_positions),
                                 torch.from_numpy(workload.global_positions), table,
                                 prefix_token_count=workload.prefix_token_count,
                                 rotary_dim=workload.rotary_dim, is_neox_style=True)
    r1_torch.scatter_rows(keys, values, torch.from_numpy(repair_slots), repaired_k, repaired_v)

    remapped = workload.tokens - workload.prefix_token_count
    assert remapped > 0  # the link rotates
    for layer in range(layers):
        got_k = _bits(keys[layer])[workload.destination_slots]
        got_v = _bits(values[layer])[workload.destination_slots]
        assert np.array_equal(got_k, expected_k[layer]), f"K of layer {layer}"
        assert np.array_equal(got_v, expected_v[layer]), f"V of layer {layer}"
        assert np.array_equal(_bits(keys[layer])[untouched], before_k[layer]), f"K rows outside, layer {layer}"
        assert np.array_equal(_bits(values[layer])[untouched], before_v[layer]), f"V rows outside, layer {layer}"
    # The prefix is a bit copy, the rest is rotated: K past the prefix differs
    # from its (unchanged) source rows in most elements.
    first = workload.prefix_token_count
    moved = _bits(keys[0])[workload.destination_slots]
    sources = _bits(keys[0])[workload.source_slots]
    assert np.array_equal(moved[:first], sources[:first])
    assert (moved[first:] != sources[first:]).mean() > 0.5
