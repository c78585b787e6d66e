"""Pins of the CPU oracle (no GPU); the rounding branches beyond the fused
fp32-table path are pinned in test_oracle_rounding_pins.py.

The oracle is trusted only because of these checks:
* conversions against library routines (torch bf16 cast, numpy fp16 cast);
* the C and numpy restatements against each other, bit for bit;
* geometry: re-rotation l -> g equals a direct fp64 rotation to g (an
  independent computation from the angles, not from the delta formula);
* rounding: the fused semantics round once (error <= 1/2 bf16 ulp of the
  exact result up to fp32 noise), which the eager semantics do not;
* planted mistakes (wrong direction, wrong pairing, dropped sin term, double
  rounding) are caught by those checks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_link_oracle as ko
from oracle import r1_torch
from legolink_amd.rope import build_cos_sin_cache
from tests import rope_math

SEED = 20260824


# ---------------------------------------------------------------------------
# Conversions.
# ---------------------------------------------------------------------------
def _interesting_f32() -> np.ndarray:
    rng = np.random.default_rng(SEED)
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7FFFFFFF) <= 0x7F800000]  # finite and inf, no NaN
    edge_bits = np.array(
        [
            0x00000000, 0x80000000, 0x3F800000, 0xBF800000, 0x7F800000, 0xFF800000,
            0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x00800000, 0x00000001,
            0x00008000, 0x00018000, 0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000,
            0x3F807FFF, 0x3F808001, 0x477FE000, 0x477FEFFF, 0x477FF000, 0x38800000,
            0x387FFFFF, 0x33000000, 0x33000001, 0x32FFFFFF, 0x33800000, 0x33C00000,
            0x38000000, 0x37FFFFFF, 0x3F801000, 0x3F803000, 0x3F802000,
        ],
        dtype=np.uint32,
    )
    return np.concatenate((bits, edge_bits)).view(np.float32)


def test_bf16_rounding_matches_torch_cast():
    values = _interesting_f32()
    expected = torch.from_numpy(values.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ko.f32_to_bf16_bits(values), expected)
    assert np.array_equal(ko.c_f32_to_bf16_bits(values), expected)


def test_bf16_rounding_of_nan_is_quiet_nan():
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FFFFFFF], dtype=np.uint32).view(np.float32)
    for out in (ko.f32_to_bf16_bits(nans), ko.c_f32_to_bf16_bits(nans)):
        assert np.all(out == 0x7FC0)
    torch_out = torch.from_numpy(nans.copy()).to(torch.bfloat16).float().numpy()
    assert np.all(np.isnan(torch_out))


def test_f16_rounding_matches_numpy_cast():
    values = _interesting_f32()
    expected = values.astype(np.float16).view(np.uint16)
    assert np.array_equal(ko.c_f32_to_f16_bits(values), expected)
    assert np.array_equal(ko.f32_to_f16_bits(values), expected)


def test_f16_widening_matches_numpy_for_every_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    actual = ko.c_f16_bits_to_f32(bits)
    finite = ~np.isnan(expected)
    assert np.array_equal(actual[finite].view(np.uint32), expected[finite].view(np.uint32))
    assert np.all(np.isnan(actual[~finite]))


# ---------------------------------------------------------------------------
# Restatements agree.
# ---------------------------------------------------------------------------
def _case(
    *,
    key_dtype: int,
    cache_dtype: int,
    tokens: int = 96,
    heads: int = 3,
    head_dim: int = 64,
    rotary_dim: int = 64,
    max_position: int = 70_000,
    theta: float = 1e6,
    seed: int = SEED,
):
    rng = np.random.default_rng(seed)
    raw = rng.standard_normal((tokens, heads, head_dim)).astype(np.float32)
    rows = ko.f32_to_bf16_bits(raw) if key_dtype == ko.BF16 else ko.f32_to_f16_bits(raw)
    local = rng.integers(0, max_position, size=tokens)
    global_ = rng.integers(0, max_position, size=tokens)
    table = build_cos_sin_cache(max_position, rotary_dim, theta=theta).numpy()
    if cache_dtype == ko.BF16:
        cache = ko.f32_to_bf16_bits(table)
    elif cache_dtype == ko.F16:
        cache = ko.f32_to_f16_bits(table)
    else:
        cache = table
    return rows, local, global_, cache


@pytest.mark.parametrize("key_dtype", [ko.BF16, ko.F16])
@pytest.mark.parametrize("cache_dtype", [ko.F32, ko.BF16, ko.F16])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rotary_dim,prefix", [(64, 0), (32, 17), (64, 96)])
@pytest.mark.parametrize("rounding", [ko.FUSED, ko.EAGER])
def test_c_and_numpy_restatements_agree(key_dtype, cache_dtype, neox, rotary_dim, prefix, rounding):
    rows, local, global_, cache = _case(
        key_dtype=key_dtype, cache_dtype=cache_dtype, rotary_dim=rotary_dim
    )
    kwargs = dict(
        key_dtype=key_dtype, cache_dtype=cache_dtype, rotary_dim=rotary_dim, neox=neox, prefix=prefix,
        rounding=rounding,
    )
    from_c = ko.rerotate_rows_c(rows, local, global_, cache, **kwargs)
    from_numpy = ko.rerotate_rows_numpy(rows, local, global_, cache, **kwargs)
    assert np.array_equal(from_c, from_numpy)
    # Prefix rows and pass-through dims are bit copies.
    assert np.array_equal(from_c[:prefix], rows[:prefix])
    assert np.array_equal(from_c[:, :, rotary_dim:], rows[:, :, rotary_dim:])


def test_restatements_agree_on_a_strided_cache():
    rows, local, global_, cache = _case(key_dtype=ko.BF16, cache_dtype=ko.F32, max_position=5000)
    wide = np.zeros((cache.shape[0], 2 * cache.shape[1] + 8), dtype=np.float32)
    wide[:, 3 : 3 + 2 * cache.shape[1] : 2] = cache
    strided = wide[:, 3 : 3 + 2 * cache.shape[1] : 2]
    assert not strided.flags.c_contiguous
    kwargs = dict(key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=64, neox=True, prefix=0)
    assert np.array_equal(
        ko.rerotate_rows_c(rows, local, global_, strided, **kwargs),
        ko.rerotate_rows_c(rows, local, global_, cache, **kwargs),
    )


def test_out_of_range_position_is_rejected():
    rows, local, global_, cache = _case(key_dtype=ko.BF16, cache_dtype=ko.F32, max_position=1000)
    local = local.copy()
    local[5] = cache.shape[0]
    with pytest.raises(IndexError):
        ko.rerotate_rows_c(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.F32,
                           rotary_dim=64, neox=True, prefix=0)


# ---------------------------------------------------------------------------
# Geometry pin: re-rotation equals a direct rotation (fp64, from angles).
# ---------------------------------------------------------------------------
def _geometry_error(rerotate, *, neox: bool, rotary_dim: int = 128, head_dim: int = 128,
                    theta: float = 1e6, tokens: int = 512, heads: int = 4, max_position: int = 2048,
                    cache_override=None) -> np.ndarray:
    """Max over elements of |rerotated - direct| / (|x1| + |x2| + 1e-3) using fp16 keys."""

    rng = np.random.default_rng(SEED + 1)
    raw = rng.standard_normal((tokens, heads, head_dim))
    local = rng.integers(0, max_position, size=tokens)
    global_ = rng.integers(0, max_position, size=tokens)
    table = build_cos_sin_cache(max_position, rotary_dim, theta=theta).numpy()
    if cache_override is not None:
        table = cache_override(table)
    keys_local = rope_math.rotate(raw, local, rotary_dim, theta=theta, neox=neox)
    rows = ko.f32_to_f16_bits(keys_local.astype(np.float32))
    out = rerotate(rows, local, global_, table, key_dtype=ko.F16, cache_dtype=ko.F32,
                   rotary_dim=rotary_dim, neox=neox, prefix=0)
    got = ko.f16_bits_to_f32(out).astype(np.float64)
    want = rope_math.rotate(raw, global_, rotary_dim, theta=theta, neox=neox)
    d1, d2 = rope_math.pair_dims(rotary_dim, neox)
    scale = np.abs(raw[:, :, d1]) + np.abs(raw[:, :, d2]) + 1e-3
    err = np.maximum(np.abs(got[:, :, d1] - want[:, :, d1]), np.abs(got[:, :, d2] - want[:, :, d2])) / scale
    return err


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rerotate", [ko.rerotate_rows_c, ko.rerotate_rows_numpy])
def test_rerotation_matches_direct_rotation(neox, rerotate):
    # fp16 key quantisation (2^-11 relative, twice) plus fp32 table angles
    # (<= 2048 * 2^-24 rad) bound the error well below 5e-3.
    assert _geometry_error(rerotate, neox=neox).max() < 5e-3


def test_partial_rotary_rerotation_matches_direct_rotation():
    assert _geometry_error(ko.rerotate_rows_c, neox=True, rotary_dim=64, head_dim=128).max() < 5e-3


def test_geometry_pin_catches_planted_mistakes():
    def swapped_direction(rows, local, global_, cache, **kw):
        return ko.rerotate_rows_numpy(rows, global_, local, cache, **kw)

    def wrong_pairing(rows, local, global_, cache, **kw):
        kw["neox"] = not kw["neox"]
        return ko.rerotate_rows_numpy(rows, local, global_, cache, **kw)

    def dropped_sin(table):
        table = table.copy()
        table[:, table.shape[1] // 2 :] = 0.0
        return table

    def swapped_halves(table):
        half = table.shape[1] // 2
        return np.concatenate((table[:, half:], table[:, :half]), axis=1)

    assert _geometry_error(swapped_direction, neox=True).max() > 0.1
    assert _geometry_error(wrong_pairing, neox=True).max() > 0.1
    assert _geometry_error(ko.rerotate_rows_numpy, neox=True, cache_override=dropped_sin).max() > 0.1
    assert _geometry_error(ko.rerotate_rows_numpy, neox=True, cache_override=swapped_halves).max() > 0.1


# ---------------------------------------------------------------------------
# Rounding pin: bf16 K with an fp32 cache is rounded once.
# ---------------------------------------------------------------------------
def _single_rounding_excess(rows_out, rows_in, local, global_, cache, rotary_dim=128, neox=True):
    """Per element: |out - exact| - 1/2 ulp(exact), where exact is the fp64 value
    of the rotation by the fp32 table entries (products exact in fp64)."""

    half = rotary_dim // 2
    c = cache.astype(np.float64)
    lc, ls = c[local, :half][:, None, :], c[local, half:2 * half][:, None, :]
    gc, gs = c[global_, :half][:, None, :], c[global_, half:2 * half][:, None, :]
    dc = gc * lc + gs * ls
    ds = gs * lc - gc * ls
    d1, d2 = rope_math.pair_dims(rotary_dim, neox)
    x = ko.bf16_bits_to_f32(rows_in).astype(np.float64)
    x1, x2 = x[:, :, d1], x[:, :, d2]
    exact1 = x1 * dc - x2 * ds
    exact2 = x2 * dc + x1 * ds
    y = ko.bf16_bits_to_f32(rows_out).astype(np.float64)
    noise = 8 * 2.0 ** -24 * (np.abs(x1) + np.abs(x2))  # fp32 rounding of the delta and products
    ex1 = np.abs(y[:, :, d1] - exact1) - 0.5 * rope_math.bf16_ulp(exact1) - noise
    ex2 = np.abs(y[:, :, d2] - exact2) - 0.5 * rope_math.bf16_ulp(exact2) - noise
    return np.maximum(ex1, ex2)


def test_fused_semantics_round_once_and_eager_semantics_do_not():
    rows, local, global_, cache = _case(
        key_dtype=ko.BF16, cache_dtype=ko.F32, tokens=512, heads=4, head_dim=128, rotary_dim=128
    )
    fused = ko.rerotate_rows_c(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.F32,
                               rotary_dim=128, neox=True, prefix=0)
    assert _single_rounding_excess(fused, rows, local, global_, cache).max() <= 0.0

    # The eager torch path (rounding after every op) is measurably different:
    # this is the planted "double rounding" mistake for the fused semantics.
    key = torch.from_numpy(rows.view(np.int16).copy()).view(torch.bfloat16)
    eager = r1_torch.remap_key_positions(
        key, torch.from_numpy(local), torch.from_numpy(global_), torch.from_numpy(cache), 128, True
    )
    eager_bits = eager.view(torch.int16).numpy().view(np.uint16)
    assert _single_rounding_excess(eager_bits, rows, local, global_, cache).max() > 0.0


# ---------------------------------------------------------------------------
# The cos/sin table recipe.
# ---------------------------------------------------------------------------
def test_cos_sin_table_follows_the_recipe():
    rotary_dim, theta, positions = 128, 1e6, 65_536
    table = build_cos_sin_cache(positions, rotary_dim, theta=theta).numpy().astype(np.float64)
    inv_freq = (1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))).numpy()
    angles32 = (np.arange(positions, dtype=np.float32)[:, None] * inv_freq[None, :]).astype(np.float64)
    half = rotary_dim // 2
    # cos/sin of the fp32 angles, to fp32 accuracy.
    assert np.abs(table[:, :half] - np.cos(angles32)).max() < 4e-7
    assert np.abs(table[:, half:] - np.sin(angles32)).max() < 4e-7
    # and of the true angles, within the fp32 angle error: inv_freq and the
    # product p * inv_freq are each rounded to fp32 (a few 2^-24 relative).
    true_angles = np.arange(positions, dtype=np.float64)[:, None] * rope_math.inv_freq64(rotary_dim, theta)[None, :]
    bound = true_angles * 2.0 ** -21 + 1e-6
    assert np.all(np.abs(table[:, :half] - np.cos(true_angles)) <= bound)
    assert np.all(np.abs(table[:, half:] - np.sin(true_angles)) <= bound)
