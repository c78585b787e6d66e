"""Invariants of the five seeded link workloads (host arrays only)."""

from __future__ import annotations

import numpy as np
import pytest

from legolink_amd.workloads import QWEN25_7B, QWEN3_32B, make_workload

EXPECTED = {
    # name: (shape, pool slots, linked tokens, repair rows, blocks)
    "c1": (QWEN25_7B, 65_536, 2_048, 24, 4),
    "c2": (QWEN25_7B, 262_144, 32_768, 240, 16),
    "c3": (QWEN25_7B, 1_048_576, 524_288, 64 * 7 * 8, 512),
    "c4": (QWEN3_32B, 131_072, 16_384, 176, 12),
    "c5": (QWEN25_7B, 262_144, 32_768, 16_352, 512),
}


@pytest.fixture(scope="module", params=sorted(EXPECTED))
def workload(request):
    return make_workload(request.param)


def test_sizes(workload):
    shape, slots, tokens, repair_rows, blocks = EXPECTED[workload.name]
    assert workload.shape == shape
    assert workload.num_slots == slots
    assert workload.tokens == tokens == sum(workload.block_lengths)
    assert workload.repair_rows == repair_rows
    assert len(workload.block_lengths) == blocks


def test_slots_are_in_range_and_disjoint(workload):
    src, dst = workload.source_slots, workload.destination_slots
    assert src.min() >= 0 and src.max() < workload.num_slots
    assert dst.min() >= 0 and dst.max() < workload.num_slots
    assert np.unique(dst).size == dst.size
    assert np.intersect1d(src, dst).size == 0
    if workload.name != "c3":  # c3 links shared blocks several times
        assert np.unique(src).size == src.size


def test_positions_and_prefix(workload):
    local, glob = workload.local_positions, workload.global_positions
    assert local.min() >= 0 and glob.min() >= 0
    assert workload.max_position < 70_000
    start = 0
    for length in workload.block_lengths:
        delta = glob[start : start + length] - local[start : start + length]
        assert np.all(delta == delta[0])  # one delta per block
        assert np.all(np.diff(glob[start : start + length]) == 1)
        start += length
    first = workload.block_lengths[0]
    identity = bool(np.all(local[:first] == glob[:first]))
    assert workload.prefix_token_count == (first if identity else 0)


def test_repair_rows_are_the_first_tokens_of_every_later_block(workload):
    per_seam = workload.notes["imp_per_seam"]
    expected = np.zeros(workload.tokens, dtype=np.uint8)
    start = 0
    blocks_per_request = len(workload.block_lengths) // workload.requests
    for index, length in enumerate(workload.block_lengths):
        if index % blocks_per_request:
            expected[start : start + min(per_seam, length)] = 1
        start += length
    assert np.array_equal(workload.repair_mask, expected)


def test_algorithmic_bytes():
    c2 = make_workload("c2")
    # 28 layers x (K + V) x 1024-byte rows, read and written: 114,688 bytes per token.
    assert c2.shape.bytes_per_token == 114_688
    assert c2.algorithmic_bytes()["total_bytes"] == 32_768 * 114_688
    c4 = make_workload("c4")
    assert c4.shape.bytes_per_token == 524_288


def test_rank_share_keeps_tokens_and_divides_heads():
    c4 = make_workload("c4")
    for tp in (1, 2, 4, 8):
        share = c4.rank_share(tp)
        assert share.shape.kv_heads == 8 // tp and share.shape.layers == 64
        assert np.array_equal(share.source_slots, c4.source_slots)
        assert np.array_equal(share.global_positions, c4.global_positions)
        assert share.algorithmic_bytes()["total_bytes"] * tp == c4.algorithmic_bytes()["total_bytes"]
    with pytest.raises(ValueError, match="must divide"):
        c4.rank_share(3)
    with pytest.raises(ValueError, match="must divide"):
        make_workload("c2").rank_share(8)


def test_block_length_ranges():
    assert all(256 <= n <= 4096 for n in make_workload("c2").block_lengths)
    assert all(512 <= n <= 2048 for n in make_workload("c4").block_lengths)


def test_workloads_are_deterministic():
    a, b = make_workload("c2"), make_workload("c2")
    assert np.array_equal(a.source_slots, b.source_slots)
    assert np.array_equal(a.local_positions, b.local_positions)


def test_row_hash_of_the_gpu_tests_sees_swaps_and_equal_sum_rows():
    """The untouched-rows check of the GPU parity tests (row_checksums) is a
    weighted hash: a swap of two elements inside a row, or a row replaced by
    one with the same plain sum, changes it (checked on CPU tensors)."""

    import torch

    from tests.gpu_helpers import row_checksums

    generator = torch.Generator().manual_seed(3)
    rows = torch.randn(64, 4, 128, generator=generator).to(torch.bfloat16)
    base = row_checksums(rows)
    swapped = rows.clone()
    swapped[5, 0, 3], swapped[5, 2, 100] = rows[5, 2, 100], rows[5, 0, 3]
    assert (row_checksums(swapped) != base).tolist() == [i == 5 for i in range(64)]
    permuted = rows.clone()
    permuted[9] = rows[9].flip(-1)  # same elements, same plain sum
    assert rows[9].view(torch.int16).sum() == permuted[9].view(torch.int16).sum()
    assert row_checksums(permuted)[9] != base[9]
    assert torch.equal(row_checksums(rows, chunk=7), base)
