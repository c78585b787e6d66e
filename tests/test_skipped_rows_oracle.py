"""Known answers for the tokens a link skips (out-of-range slot or position).

The reference's fused kernel loads slots and positions unchecked
(legolink_triton.py:336-339) and its torch path raises on them; this
library's kernels skip such tokens and count them.  These hand-made cases fix
which tokens count, and that the pool-level oracle leaves their destination
rows alone while linking the rest.
"""

from __future__ import annotations

import numpy as np

from oracle import kv_link_oracle as ko

SRC_SLOTS, DST_SLOTS, CACHE_ROWS = 10, 12, 8


def _mask(src, dst, local, global_, prefix, repair_mask=None):
    return ko.skipped_token_mask(src, dst, local, global_, source_slots=SRC_SLOTS, destination_slots=DST_SLOTS,
                                 cache_rows=CACHE_ROWS, prefix=prefix, repair_mask=repair_mask)


def test_which_tokens_are_skipped():
    #         t:   0   1   2   3   4   5   6   7   8
    src = [0, 9, 10, -1, 2, 3, 4, 5, 6]
    dst = [0, 1, 2, 3, 12, -1, 6, 7, 8]
    local = [7, 9, 0, 0, 0, 0, 8, -1, 3]
    glob = [0, 0, 0, 0, 0, 0, 1, 2, 7]
    # prefix 2: tokens 0 and 1 are copied, their positions are not read.
    got = _mask(src, dst, local, glob, prefix=2)
    assert got.tolist() == [False, False, True, True, True, True, True, True, False]
    # With prefix 0, token 1's local position 9 >= 8 is out of the table.
    assert _mask(src, dst, local, glob, prefix=0).tolist()[:2] == [False, True]
    # Masked tokens are never counted, whatever their indices.
    mask = np.zeros(9, dtype=np.uint8)
    mask[[2, 6]] = 1
    assert _mask(src, dst, local, glob, prefix=2, repair_mask=mask).sum() == 4


def test_pool_link_leaves_skipped_rows_and_links_the_rest():
    rng = np.random.default_rng(5)
    heads, dim = 2, 8
    keys = [rng.integers(0, 1 << 15, size=(DST_SLOTS, heads, dim), dtype=np.uint16)]
    values = [rng.integers(0, 1 << 15, size=(DST_SLOTS, heads, dim), dtype=np.uint16)]
    cache = rng.standard_normal((CACHE_ROWS, dim)).astype(np.float32)
    src = np.array([1, 2, 30, 4])
    dst = np.array([5, 6, 7, 8])
    local = np.array([0, 1, 2, 99])
    glob = np.array([3, 4, 5, 6])
    common = dict(key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=dim, neox=True, prefix=0)
    out_k, out_v = ko.link_pool(keys, values, src, dst, local, glob, cache, **common)
    # Tokens 2 (source 30) and 3 (local 99) are skipped: rows 7 and 8 keep their bits.
    assert np.array_equal(out_k[0][[7, 8]], keys[0][[7, 8]]) and np.array_equal(out_v[0][[7, 8]], values[0][[7, 8]])
    # The others are the link of the valid tokens alone.
    good_k, good_v = ko.link_pool(keys, values, src[:2], dst[:2], local[:2], glob[:2], cache, **common)
    assert np.array_equal(out_k[0], good_k[0]) and np.array_equal(out_v[0], good_v[0])
    assert not np.array_equal(out_k[0][[5, 6]], keys[0][[5, 6]])
