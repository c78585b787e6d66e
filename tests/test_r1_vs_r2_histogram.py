"""The committed R1-vs-R2 histogram is what the oracle computes, and its
figures obey what the two roundings fix.

tests/golden/r1_vs_r2_histogram.py re-rotates the same K rows with the
reference's torch-path rounding (R1, pic_runtime.py:6025-6058 + :1868-1885)
and its fused-kernel rounding (R2, legolink_triton.py:413-470).
"""

from __future__ import annotations

import json

from tests.golden import r1_vs_r2_histogram as h


def test_committed_histogram_is_reproduced():
    assert h.histogram() == json.loads(h.OUTPUT.read_text())


def test_histogram_figures_follow_the_roundings():
    cases = {(c["case"], c["k_distribution"]): c for c in json.loads(h.OUTPUT.read_text())["cases"]}
    for distribution in h.DISTRIBUTIONS:
        # With a bf16 table the fused kernel takes the bf16-rounded chain, the
        # same operations as the torch path: nothing differs.
        same = cases[("bf16 K, bf16 table", distribution)]
        assert same["share_differing"] == 0 and same["max_ulp_apart"] == 0
        for name in ("bf16 K, fp32 table", "fp16 K, fp32 table"):
            case = cases[(name, distribution)]
            assert sum(case["ulp_apart"].values()) == case["elements"] == h.TOKENS * h.HEADS * h.DIM
            # R2 rounds an fp32 result once: correctly rounded but where fp32
            # error meets a rounding boundary, within 1/2 ulp of the pair norm
            # plus fp32 noise.
            r2 = case["error_vs_exact"]["R2"]
            assert r2["correctly_rounded_share"] >= 0.999 and r2["max_pair_norm_ulps"] <= 0.51
            # R1 rounds every product: a third of the elements move, some by
            # more than one ulp.
            r1 = case["error_vs_exact"]["R1"]
            assert 0.2 < case["share_differing"] < 0.5 and 0.02 < case["share_more_than_1_ulp"] < 0.1
            assert r1["correctly_rounded_share"] < 0.8 and 1.0 < r1["max_pair_norm_ulps"] < 3.0
