"""GPU checks of the visit ordering of a map set (ll_order_link_maps), by
destination or by source slot: the output is a permutation of the input
entries that keeps the identity prefix in place and lists the rest by bucket
of the key slots (by slot where the pool has at most 16,384 rows); masks
follow their entries; duplicate and out-of-range slots still give a
permutation; the shared workspace is zero again after every call."""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from legolink_amd import _native, link_maps
from tests.gpu_helpers import report

pytestmark = pytest.mark.gpu


def _maps(rng, n, num_slots, *, duplicates=False, outside=False):
    if duplicates:
        dst = rng.integers(0, num_slots, size=n)
    else:
        dst = rng.permutation(num_slots)[:n] if n <= num_slots else rng.integers(0, num_slots, size=n)
    dst = dst.astype(np.int64)
    if outside:
        pick = rng.choice(n, size=max(1, n // 50), replace=False)
        dst[pick] = rng.choice([-1, -(1 << 40), num_slots, num_slots + 12345, 1 << 50], size=pick.size)
    src = rng.integers(0, 1 << 40, size=n)
    local = rng.integers(0, 1 << 20, size=n)
    glob = np.arange(n, dtype=np.int64) * 3 + 1  # distinct: identifies each entry
    return np.stack([src, dst, local, glob]).astype(np.int64)


def _bucket(slots, num_slots):
    shift = 0
    while ((num_slots - 1) >> shift) >= _native.ORDER_BUCKETS:
        shift += 1
    return np.where(slots < 0, 0, np.where(slots >= num_slots, _native.ORDER_BUCKETS - 1, slots >> shift))


CASES = [
    # name, entries, prefix, pool rows, duplicates, outside, mask
    ("small_pool_exact", 5000, 0, 12000, False, False, False),
    ("qwen_pool_with_prefix", 32512, 64, 262144, False, False, True),
    ("large_pool", 40000, 1000, 1 << 22, False, False, False),
    ("duplicates", 20000, 17, 8192, True, False, True),
    ("outside_the_pool", 20000, 0, 262144, False, True, False),
    ("all_prefix", 3000, 3000, 1000, False, False, True),
    ("one_entry_tail", 2, 1, 100, False, False, False),
]


@pytest.mark.parametrize("key_row", [1, 0], ids=["by_destination", "by_source"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_order_is_a_bucketed_permutation(gpu_device, case, key_row):
    name, n, prefix, num_slots, duplicates, outside, with_mask = case
    rng = np.random.default_rng(zlib.crc32(name.encode()) + key_row)
    workspace = torch.zeros(_native.ORDER_WORKSPACE_BYTES, dtype=torch.uint8, device=gpu_device)
    for call in range(2):  # the second call reuses the workspace the first left
        entries = n if call == 0 else max(prefix, n // 3)
        host = _maps(rng, entries, num_slots, duplicates=duplicates, outside=outside)
        if key_row == 0:  # the slots to order by in the source row
            host = host[[1, 0, 2, 3]].copy()
        mask_host = rng.integers(0, 2, size=entries).astype(np.uint8) if with_mask else None
        maps = torch.from_numpy(host).to(gpu_device)
        mask = torch.from_numpy(mask_host).to(gpu_device) if with_mask else None
        report(f"order {name} call {call}: {entries} entries, prefix {prefix}, pool {num_slots}")
        out, out_mask = link_maps.order_link_maps(maps, mask, key_row=key_row, prefix=prefix,
                                                  num_slots=num_slots, workspace=workspace)
        torch.cuda.synchronize(gpu_device)
        got = out.cpu().numpy()
        assert np.array_equal(got[:, :prefix], host[:, :prefix])
        # A permutation of the tail: every entry (its global position is unique) once.
        order = np.argsort(host[3, prefix:])
        got_order = np.argsort(got[3, prefix:])
        assert np.array_equal(host[:, prefix:][:, order], got[:, prefix:][:, got_order])
        buckets = _bucket(got[key_row, prefix:], num_slots)
        assert (np.diff(buckets) >= 0).all(), "tail not in bucket order"
        if num_slots <= _native.ORDER_BUCKETS and not outside:
            assert (np.diff(got[key_row, prefix:]) >= 0).all()
        if with_mask:
            by_position = dict(zip(host[3].tolist(), mask_host.tolist()))
            assert out_mask.cpu().numpy().tolist() == [by_position[g] for g in got[3].tolist()]
        counters = workspace.view(torch.int32)
        assert int(counters[: _native.ORDER_BUCKETS].count_nonzero()) == 0, "bucket counts not cleared"
