"""Seeded random links on the GPU against the oracle.

Every case draws a shape (heads, key / value / rotary dims), dtypes (K/V,
cos/sin table, each map's index type), neox or GPT-J pairs, a layer count
(up to two launches), a prefix, a repair mask, a separate source pool or
not, the rounding, the delta placement, streamed or cached row loads, and
possibly out-of-range slots and positions; the pools after the link must
equal the oracle's bit for bit and the skipped-token counter must equal the
oracle's count.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from legolink_amd import _native, kv_link
from legolink_amd.rope import build_cos_sin_cache
from oracle import kv_link_oracle as ko
from tests.gpu_helpers import TORCH_TO_CODE, bits, cache_host, make_pool, report

pytestmark = pytest.mark.gpu

SHAPES = [  # key dim, value dim, rotary dim
    (128, 128, 128), (128, 128, 64), (64, 64, 64), (256, 256, 256), (256, 256, 128),
    (32, 32, 32), (32, 32, 16), (128, 64, 128), (40, 24, 16), (128, 128, 32),
]
MAX_POSITION = 6000


def _case(seed: int) -> dict:
    rng = np.random.default_rng([20261202, seed])
    kdim, vdim, rotary = SHAPES[int(rng.integers(len(SHAPES)))]
    index_kind = int(rng.integers(3))
    return {
        "heads": int(rng.choice([1, 2, 3, 4, 8])),
        "kdim": kdim, "vdim": vdim, "rotary": rotary,
        "dtype": [torch.bfloat16, torch.float16][int(rng.integers(2))],
        "cache_dtype": [torch.float32, torch.float32, torch.bfloat16, torch.float16][int(rng.integers(4))],
        "neox": bool(rng.random() < 0.7),
        "index": ([torch.int64] * 4 if index_kind == 0 else [torch.int32] * 4 if index_kind == 1 else
                  [[torch.int32, torch.int64][int(rng.integers(2))] for _ in range(4)]),
        "layers": int(rng.choice([1, 2, 3, 5, 28, 65, 70])),
        "tokens": int(rng.integers(1, 400)),
        "prefix_share": float(rng.choice([0.0, 0.0, rng.random(), 1.0])),
        "mask": float(rng.choice([0.0, 0.0, 0.1, 0.5])),
        "bool_mask": bool(rng.random() < 0.3),
        "separate_source": bool(rng.random() < 0.25),
        "rounding": ["fused", "eager"][int(rng.integers(2))],
        "delta_staging": ["auto", "per_wave", "workgroup"][int(rng.integers(3))],
        "stream": bool(rng.random() < 0.5),
        "generic": bool(rng.random() < 0.15),
        "corrupt": float(rng.choice([0.0, 0.0, 0.1])),
        "rng": rng,
    }


@pytest.mark.parametrize("seed", range(256))
def test_random_link_matches_oracle(gpu_device, seed):
    c = _case(seed)
    rng = c.pop("rng")
    report(f"fuzz {seed}: " + ", ".join(f"{k}={v}" for k, v in c.items()))
    tokens, heads = c["tokens"], c["heads"]
    slots = 2 * tokens + 37
    source_slots_count = tokens + 23 if c["separate_source"] else slots
    perm = rng.permutation(slots)
    dst = perm[:tokens]
    src = (rng.permutation(source_slots_count)[:tokens] if c["separate_source"] else perm[tokens:2 * tokens])
    local = rng.integers(0, MAX_POSITION, size=tokens)
    glob = rng.integers(0, MAX_POSITION, size=tokens)
    prefix = int(round(c["prefix_share"] * tokens))
    mask_np = (rng.random(tokens) < c["mask"]).astype(np.uint8) if c["mask"] else None
    skipped = None
    if c["corrupt"]:
        for t in np.flatnonzero(rng.random(tokens) < c["corrupt"]):
            which = int(rng.integers(4))
            target = (src, dst, local, glob)[which]
            limit = (source_slots_count, slots, MAX_POSITION, MAX_POSITION)[which]
            target[t] = -1 - int(rng.integers(2)) if rng.random() < 0.5 else limit + int(rng.integers(3))
        skipped = torch.zeros(1, dtype=torch.int64, device=gpu_device)
    keys, values = make_pool(c["layers"], slots, heads, c["kdim"], c["vdim"], c["dtype"], gpu_device, seed)
    source_keys = source_values = None
    if c["separate_source"]:
        source_keys, source_values = make_pool(c["layers"], source_slots_count, heads, c["kdim"], c["vdim"],
                                               c["dtype"], gpu_device, seed + 1000)
    table = build_cos_sin_cache(MAX_POSITION, c["rotary"], theta=1e6).to(c["cache_dtype"])
    maps = [torch.from_numpy(np.ascontiguousarray(a)).to(d).to(gpu_device)
            for a, d in zip((src, dst, local, glob), c["index"])]
    mask = None
    if mask_np is not None:
        mask = torch.from_numpy(mask_np).to(gpu_device)
        if c["bool_mask"]:
            mask = mask.bool()
    want_k, want_v = ko.link_pool(
        [bits(k) for k in keys], [bits(v) for v in values], src, dst, local, glob, cache_host(table),
        key_dtype=TORCH_TO_CODE[c["dtype"]], cache_dtype=TORCH_TO_CODE[c["cache_dtype"]],
        rotary_dim=c["rotary"], neox=c["neox"], prefix=prefix, repair_mask=mask_np,
        source_key_layers=None if source_keys is None else [bits(k) for k in source_keys],
        source_value_layers=None if source_values is None else [bits(v) for v in source_values],
        rounding=ko.EAGER if c["rounding"] == "eager" else ko.FUSED)
    kv_link.fused_kv_link_layers_inplace(
        key_buffers=keys, value_buffers=values, source_slots=maps[0], destination_slots=maps[1],
        local_positions=maps[2], global_positions=maps[3], cos_sin_cache=table.to(gpu_device),
        prefix_token_count=prefix, rotary_dim=c["rotary"], is_neox_style=c["neox"], repair_mask=mask,
        kernel=_native.KERNEL_GENERIC if c["generic"] else _native.KERNEL_AUTO,
        source_key_buffers=source_keys, source_value_buffers=source_values,
        stream_source_rows=c["stream"], rounding=c["rounding"], delta_staging=c["delta_staging"],
        skipped_rows=skipped)
    torch.cuda.synchronize(gpu_device)
    for layer in range(c["layers"]):
        assert np.array_equal(bits(values[layer]), want_v[layer]), f"seed {seed}: V layer {layer}"
        diff = np.argwhere(bits(keys[layer]) != want_k[layer])
        assert diff.size == 0, f"seed {seed}: K layer {layer} differs at {diff[:4].tolist()}"
    if skipped is not None:
        expected = ko.skipped_token_mask(src, dst, local, glob, source_slots=source_slots_count,
                                         destination_slots=slots, cache_rows=MAX_POSITION, prefix=prefix,
                                         repair_mask=mask_np)
        assert int(skipped.item()) == int(expected.sum()), f"seed {seed}: skipped-token count"
