"""How far the reference's two K re-rotation roundings are apart, in ulps.

The reference re-rotates a linked block's K in one of two ways:

* R2, its fused Triton kernel (patched_sglang_files/python/sglang/srt/
  legolink_triton.py:413-470): the delta and the rotation in fp32, one
  rounding to the key dtype at the store (with a 16-bit table and bf16 K,
  the bf16-rounded chain of :437-468);
* R1, its torch path (pic_runtime.py:6025-6058 with _apply_rotary_emb,
  :1868-1885): the delta in the table's dtype, cast to the key dtype, then
  every product and sum rounded to the key dtype.

The reference runs R1 by default (SGLANG_PIC_TRITON_FUSED_KV_LINK "0"), for
links with clone blocks and for promotion, and R2 when the fused kernel is
enabled.  This script re-rotates the same rows both ways with the oracle (C
restatement, ``rounding`` FUSED / EAGER) and reports, per case:

* the histogram of |R1 - R2| in ulps of the key dtype (distance between the
  16-bit patterns in value order; +0 and -0 are 0 apart), and the share more
  than 1 ulp apart measured as |a - b| in ulps at max(|a|, |b|);
* each rounding's error against the exact rotation by the table's entries
  (fp64): the share of elements within 1/2 ulp of the exact value
  (correctly rounded), and the largest and mean error in ulps of the pair's
  norm (a rotation keeps it; an element near zero after cancellation would
  make ulps of the element itself meaningless).

Inputs (seeded): 4,096 tokens x 4 KV heads x 128 dims (Qwen2.5-7B's K
rows), neox, rotary_dim 128, theta 1e6; tokens in blocks of 512 compiled at
local positions 0..511 and linked at random starts in a 32,768-position
request.  K elements are N(0, 1) ("normal") or N(0, 1) times a per-channel
scale log-uniform in [0.05, 20] ("outlier_channels", as model K rows have).
The output is committed as r1_vs_r2_histogram.json; the test
tests/test_r1_vs_r2_histogram.py recomputes it and compares.

    python tests/golden/r1_vs_r2_histogram.py        (rewrites the JSON)
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

REPO_ROOT = Path(__file__).resolve().parents[2]
if str(REPO_ROOT) not in sys.path:
    sys.path.insert(0, str(REPO_ROOT))

from oracle import kv_link_oracle as ko  # noqa: E402

OUTPUT = Path(__file__).resolve().parent / "r1_vs_r2_histogram.json"
TOKENS, HEADS, DIM, BLOCK, REQUEST = 4096, 4, 128, 512, 32768
THETA = 1e6
SEED = 20261202
BUCKETS = ((0, 0), (1, 1), (2, 2), (3, 4), (5, 8), (9, None))
CASES = (
    ("bf16 K, fp32 table", ko.BF16, ko.F32),
    ("bf16 K, bf16 table", ko.BF16, ko.BF16),
    ("fp16 K, fp32 table", ko.F16, ko.F32),
)
DISTRIBUTIONS = ("normal", "outlier_channels")


def _table(rows: int) -> np.ndarray:
    inv_freq = 1.0 / THETA ** (np.arange(0, DIM, 2, dtype=np.float32) / np.float32(DIM))
    angles = np.outer(np.arange(rows, dtype=np.float32), inv_freq.astype(np.float32)).astype(np.float32)
    # cos/sin in fp64, then rounded: the same table on every CPU (numpy's fp32
    # cos/sin may use different vector code per machine).
    angles = angles.astype(np.float64)
    return np.concatenate([np.cos(angles), np.sin(angles)], axis=-1).astype(np.float32)


def _ordered(bits: np.ndarray) -> np.ndarray:
    """16-bit float patterns -> integers in value order (+0 and -0 both 0)."""

    bits = bits.astype(np.int64)
    magnitude = bits & 0x7FFF
    return np.where(bits & 0x8000, -magnitude, magnitude)


def _ulp(values: np.ndarray, key_dtype: int) -> np.ndarray:
    """ulp of the key dtype at |values| (normal range; subnormal floor)."""

    mantissa_bits, min_exponent = (7, -126) if key_dtype == ko.BF16 else (10, -14)
    exponent = np.floor(np.log2(np.maximum(np.abs(values), 2.0 ** min_exponent)))
    return 2.0 ** (exponent - mantissa_bits)


def _inputs(rng: np.random.Generator, distribution: str):
    starts = rng.integers(0, REQUEST - BLOCK + 1, size=TOKENS // BLOCK)
    local = np.tile(np.arange(BLOCK, dtype=np.int64), TOKENS // BLOCK)
    global_ = (np.repeat(starts, BLOCK) + local).astype(np.int64)
    values = rng.standard_normal((TOKENS, HEADS, DIM)).astype(np.float32)
    if distribution == "outlier_channels":
        values *= np.exp(rng.uniform(np.log(0.05), np.log(20.0), size=(1, HEADS, DIM))).astype(np.float32)
    return values, local, global_


def _exact(x: np.ndarray, local, global_, table: np.ndarray) -> np.ndarray:
    half = DIM // 2
    t = table.astype(np.float64)
    lc, ls = t[local, :half][:, None, :], t[local, half:][:, None, :]
    gc, gs = t[global_, :half][:, None, :], t[global_, half:][:, None, :]
    dc, ds = gc * lc + gs * ls, gs * lc - gc * ls
    x1, x2 = x[:, :, :half].astype(np.float64), x[:, :, half:].astype(np.float64)
    return np.concatenate([x1 * dc - x2 * ds, x2 * dc + x1 * ds], axis=-1)


def histogram_case(key_dtype: int, cache_dtype: int, distribution: str, seed: int = SEED) -> dict:
    rng = np.random.default_rng([seed, DISTRIBUTIONS.index(distribution)])
    values, local, global_ = _inputs(rng, distribution)
    rows = (ko.f32_to_bf16_bits if key_dtype == ko.BF16 else ko.f32_to_f16_bits)(values)
    table32 = _table(REQUEST)
    cache = table32 if cache_dtype == ko.F32 else (
        ko.f32_to_bf16_bits(table32) if cache_dtype == ko.BF16 else ko.f32_to_f16_bits(table32))
    common = dict(key_dtype=key_dtype, cache_dtype=cache_dtype, rotary_dim=DIM, neox=True, prefix=0)
    r2 = ko.rerotate_rows_c(rows, local, global_, cache, rounding=ko.FUSED, **common)
    r1 = ko.rerotate_rows_c(rows, local, global_, cache, rounding=ko.EAGER, **common)
    apart = np.abs(_ordered(r1) - _ordered(r2)).reshape(-1)
    total = int(apart.size)
    buckets = {}
    for low, high in BUCKETS:
        label = f"{low}" if low == high else (f"{low}-{high}" if high is not None else f">={low}")
        inside = (apart >= low) if high is None else ((apart >= low) & (apart <= high))
        buckets[label] = int(np.count_nonzero(inside))
    to_f32 = ko.bf16_bits_to_f32 if key_dtype == ko.BF16 else ko.f16_bits_to_f32
    # The same distance measured as |a - b| in ulps at max(|a|, |b|): a pair
    # apart by one step across a power of two counts as half an ulp or one.
    a, b = to_f32(r1).astype(np.float64).reshape(-1), to_f32(r2).astype(np.float64).reshape(-1)
    at_larger = np.abs(a - b) / _ulp(np.maximum(np.abs(a), np.abs(b)), key_dtype)
    exact = _exact(to_f32(rows), local, global_, ko.cache_to_f32(cache, cache_dtype))
    # A rotation keeps each pair's norm: errors are also measured in ulps of
    # it, which cancellation in one element of the pair does not inflate.
    half = DIM // 2
    pair_norm = np.hypot(exact[:, :, :half], exact[:, :, half:])
    pair_ulp = np.concatenate([_ulp(pair_norm, key_dtype)] * 2, axis=-1)
    errors = {}
    for name, got in (("R1", r1), ("R2", r2)):
        error = np.abs(to_f32(got).astype(np.float64) - exact)
        in_pair_ulps = error / pair_ulp
        errors[name] = {
            "correctly_rounded_share": round(float(np.mean(error <= 0.5 * _ulp(exact, key_dtype) * (1 + 1e-9))), 6),
            "max_pair_norm_ulps": round(float(in_pair_ulps.max()), 4),
            "mean_pair_norm_ulps": round(float(in_pair_ulps.mean()), 5),
        }
    return {
        "elements": total,
        "ulp_apart": buckets,
        "share_differing": round(1.0 - buckets["0"] / total, 6),
        "share_more_than_1_ulp": round(1.0 - (buckets["0"] + buckets["1"]) / total, 6),
        "max_ulp_apart": int(apart.max()),
        "share_more_than_1_ulp_at_larger": round(float(np.mean(at_larger > 1.0 + 1e-9)), 6),
        "max_ulp_at_larger": round(float(at_larger.max()), 3),
        "error_vs_exact": errors,
    }


def histogram() -> dict:
    return {
        "inputs": {"tokens": TOKENS, "kv_heads": HEADS, "head_dim": DIM, "rotary_dim": DIM, "neox": True,
                   "theta": THETA, "block_tokens": BLOCK, "request_positions": REQUEST, "seed": SEED},
        "cases": [
            {"case": name, "k_distribution": distribution,
             **histogram_case(key_dtype, cache_dtype, distribution)}
            for name, key_dtype, cache_dtype in CASES for distribution in DISTRIBUTIONS
        ],
    }


if __name__ == "__main__":
    result = histogram()
    OUTPUT.write_text(json.dumps(result, indent=1) + "\n")
    for case in result["cases"]:
        print(f"{case['case']:20s} {case['k_distribution']:17s} differ {case['share_differing']:.4f} "
              f">1ulp {case['share_more_than_1_ulp']:.4f} max {case['max_ulp_apart']} "
              f"(at larger: >1 {case['share_more_than_1_ulp_at_larger']:.4f} max {case['max_ulp_at_larger']})  "
              f"R1 exact {case['error_vs_exact']['R1']['correctly_rounded_share']:.4f} "
              f"(max {case['error_vs_exact']['R1']['max_pair_norm_ulps']})  "
              f"R2 exact {case['error_vs_exact']['R2']['correctly_rounded_share']:.4f} "
              f"(max {case['error_vs_exact']['R2']['max_pair_norm_ulps']})")
