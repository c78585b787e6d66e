"""Pins of the oracle's rounding branches beyond the fused fp32-table path (no GPU).

Eager rounding (the reference's torch path, pic_runtime.py:6039-6058 with
_apply_rotary_emb :1874-1885), restated by ``oracle/r1_torch.py`` (torch) and
by the C and numpy oracles (``rounding=EAGER``):
* the reference's own bit-exact known answer (tests/pic/test_rope_remap.py:53-78);
* its fp64 remap cases at atol 2e-5 (tests/pic/test_rope_remap.py:12-35), with
  planted direction, pairing, sign and dropped-term mistakes that must fail;
* at the Qwen shape, every element within the error budget of its rounding
  points (delta cast, products and sum each rounded to bf16);
* the C and numpy restatements equal torch bit for bit on every dtype pair.

Fused rounding with bf16 K and a 16-bit table (legolink_triton.py:437-468):
* with a bf16 table the chain is torch's own bf16 arithmetic (the reference's
  torch path computes exactly that with a bf16 table);
* with an fp16 table it is torch's mixed arithmetic (fp32 products of the
  widened entries cast to bf16, then bf16 sums and products);
* geometry: within a derived multi-rounding bound of a direct fp64 rotation
  computed from the angles, which a flipped sign, swapped pairs or a swapped
  direction break; a dropped rounding breaks the torch equality.

Fused rounding with fp16 K (legolink_triton.py:469-470): one rounding to fp16
(within 1/2 fp16 ulp of the exact rotation by the table's entries).  A
lowering that contracts the products into fused multiply-adds, as the
reference's Triton kernel may, stays within 1 fp16 ulp of it.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from legolink_amd.rope import build_cos_sin_cache
from oracle import kv_link_oracle as ko
from oracle import r1_torch
from tests import rope_math

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "reference_known_answers.json").read_text())
SEED = 20260824
TORCH_DTYPES = {ko.BF16: torch.bfloat16, ko.F16: torch.float16, ko.F32: torch.float32}
U_BF16 = 2.0 ** -8  # unit roundoff of bf16 (8 significand bits)
U_F16 = 2.0 ** -11


def _torch_tensor(array: np.ndarray, dtype: int) -> torch.Tensor:
    """uint16 bit patterns (or fp32 values for F32) as a torch tensor of ``dtype``."""

    if dtype == ko.F32:
        return torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32))
    return torch.from_numpy(np.ascontiguousarray(array).view(np.int16).copy()).view(TORCH_DTYPES[dtype])


def _bits(tensor: torch.Tensor) -> np.ndarray:
    return tensor.contiguous().view(torch.int16).numpy().view(np.uint16)


def _table(max_position: int, rotary_dim: int, theta: float, dtype: int) -> np.ndarray:
    table = build_cos_sin_cache(max_position, rotary_dim, theta=theta).numpy()
    if dtype == ko.BF16:
        return ko.f32_to_bf16_bits(table)
    if dtype == ko.F16:
        return ko.f32_to_f16_bits(table)
    return table


def _random_case(*, key_dtype, cache_dtype, tokens=256, heads=4, head_dim=128, rotary_dim=128,
                 max_position=70_000, theta=1e6, seed=SEED):
    rng = np.random.default_rng(seed)
    raw = rng.standard_normal((tokens, heads, head_dim)).astype(np.float32)
    rows = ko.f32_to_bf16_bits(raw) if key_dtype == ko.BF16 else ko.f32_to_f16_bits(raw)
    local = rng.integers(0, max_position, size=tokens)
    global_ = rng.integers(0, max_position, size=tokens)
    return rows, local, global_, _table(max_position, rotary_dim, theta, cache_dtype)


def _r1_bits(rows, local, global_, cache, *, key_dtype, cache_dtype, rotary_dim, neox, prefix=0):
    key = _torch_tensor(rows, key_dtype)
    tail = r1_torch.remap_key_positions(
        key[prefix:], torch.from_numpy(np.asarray(local[prefix:])), torch.from_numpy(np.asarray(global_[prefix:])),
        _torch_tensor(cache, cache_dtype), rotary_dim, neox)
    return np.concatenate([rows[:prefix], _bits(tail)])


# ---------------------------------------------------------------------------
# Eager rounding: the reference's known answers.
# ---------------------------------------------------------------------------
def _known_answer_inputs():
    case = GOLDEN["bf16_single_delta_rounding"]
    table = build_cos_sin_cache(case["max_position"], case["rotary_dim"], theta=case["theta"])
    key = torch.zeros(*case["key_shape"], dtype=torch.bfloat16)
    for index, value in case["key_nonzero"].items():
        key[0, 0, int(index)] = value
    return case, table, key


def test_r1_reproduces_the_reference_single_delta_rounding_answer():
    case, table, key = _known_answer_inputs()
    expected = np.array(case["expected_bits"], dtype=np.uint16)
    got = r1_torch.remap_key_positions(key, torch.tensor([case["local"]]), torch.tensor([case["destination"]]),
                                       table, case["rotary_dim"], True)
    assert np.array_equal(_bits(got).reshape(-1), expected)
    rows = _bits(key)
    for rerotate in (ko.rerotate_rows_c, ko.rerotate_rows_numpy):
        out = rerotate(rows, np.array([case["local"]]), np.array([case["destination"]]), table.numpy(),
                       key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=case["rotary_dim"], neox=True,
                       prefix=0, rounding=ko.EAGER)
        assert np.array_equal(out.reshape(-1), expected)


def test_known_answer_separates_the_two_roundings():
    # The reference keeps this input because one rounding of the rotation
    # (fused) and the eager chain give different bf16 results here.
    case, table, key = _known_answer_inputs()
    fused = ko.rerotate_rows_c(_bits(key), np.array([case["local"]]), np.array([case["destination"]]),
                               table.numpy(), key_dtype=ko.BF16, cache_dtype=ko.F32,
                               rotary_dim=case["rotary_dim"], neox=True, prefix=0, rounding=ko.FUSED)
    assert not np.array_equal(fused.reshape(-1), np.array(case["expected_bits"], dtype=np.uint16))


def _remap_case_error(case, remap) -> float:
    """Max |remap(local key) - direct rotation to the destination| of one of the
    reference's fp64 remap cases (fp32 keys, as the reference's test uses)."""

    spec = GOLDEN["rope_remap_cases"]
    raw = torch.randn(4, spec["heads"], spec["rotary_dim"], generator=torch.Generator().manual_seed(SEED))
    local = np.array(case["local"])
    destination = np.array(case["destination"])
    theta = spec["theta"]
    local_key = torch.from_numpy(rope_math.rotate(raw.double().numpy(), local, spec["rotary_dim"], theta=theta)).float()
    table = build_cos_sin_cache(spec["max_position"], spec["rotary_dim"], theta=theta)
    got = remap(local_key, torch.from_numpy(local), torch.from_numpy(destination), table).double().numpy()
    want = rope_math.rotate(raw.double().numpy(), destination, spec["rotary_dim"], theta=theta)
    return float((np.abs(got - want) - spec["atol"] * np.abs(want)).max())


@pytest.mark.parametrize("index", range(len(GOLDEN["rope_remap_cases"]["cases"])))
def test_r1_remap_matches_the_reference_fp64_cases(index):
    spec = GOLDEN["rope_remap_cases"]
    case = spec["cases"][index]
    error = _remap_case_error(case, lambda key, lp, gp, table: r1_torch.remap_key_positions(
        key, lp, gp, table, spec["rotary_dim"], True))
    assert error <= spec["atol"]


def test_fp64_remap_cases_catch_planted_mistakes():
    spec = GOLDEN["rope_remap_cases"]
    rotary = spec["rotary_dim"]
    half = rotary // 2

    def negated_sin(table):
        table = table.clone()
        table[:, half:] *= -1
        return table

    def dropped_sin(table):
        table = table.clone()
        table[:, half:] = 0
        return table

    planted = {
        "direction": lambda k, lp, gp, t: r1_torch.remap_key_positions(k, gp, lp, t, rotary, True),
        "pairing": lambda k, lp, gp, t: r1_torch.remap_key_positions(k, lp, gp, t, rotary, False),
        "sign": lambda k, lp, gp, t: r1_torch.remap_key_positions(k, lp, gp, negated_sin(t), rotary, True),
        "dropped_sin": lambda k, lp, gp, t: r1_torch.remap_key_positions(k, lp, gp, dropped_sin(t), rotary, True),
    }
    for name, remap in planted.items():
        worst = max(_remap_case_error(case, remap) for case in spec["cases"])
        assert worst > 100 * spec["atol"], name


# ---------------------------------------------------------------------------
# Eager rounding at the Qwen shape.
# ---------------------------------------------------------------------------
def _exact_from_table(rows, local, global_, cache, *, key_dtype, cache_dtype, rotary_dim=128, neox=True):
    """fp64 rotation by the table's own entries (products exact in fp64)."""

    half = rotary_dim // 2
    c = ko.cache_to_f32(cache, cache_dtype).astype(np.float64)
    lc, ls = c[local, :half][:, None, :], c[local, half:2 * half][:, None, :]
    gc, gs = c[global_, :half][:, None, :], c[global_, half:2 * half][:, None, :]
    dc = gc * lc + gs * ls
    ds = gs * lc - gc * ls
    d1, d2 = rope_math.pair_dims(rotary_dim, neox)
    to_f32 = ko.bf16_bits_to_f32 if key_dtype == ko.BF16 else ko.f16_bits_to_f32
    x = to_f32(rows).astype(np.float64)
    x1, x2 = x[:, :, d1], x[:, :, d2]
    return x1, x2, dc, ds, x1 * dc - x2 * ds, x2 * dc + x1 * ds, (d1, d2)


def test_r1_bf16_stays_within_the_budget_of_its_rounding_points():
    rows, local, global_, cache = _random_case(key_dtype=ko.BF16, cache_dtype=ko.F32, tokens=512)
    eager = _r1_bits(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.F32, rotary_dim=128, neox=True)
    x1, x2, dc, ds, exact1, exact2, (d1, d2) = _exact_from_table(rows, local, global_, cache,
                                                                 key_dtype=ko.BF16, cache_dtype=ko.F32)
    got = ko.bf16_bits_to_f32(eager).astype(np.float64)
    # delta cast to bf16 (u), products rounded (u), sum rounded (u), plus the
    # fp32 delta (a few 2^-24); |o| <= |x1 dc| + |x2 ds| bounds the last term.
    terms = np.abs(x1 * dc) + np.abs(x2 * ds)
    cross = np.abs(x2 * dc) + np.abs(x1 * ds)
    noise = 8 * 2.0 ** -24 * (np.abs(x1) + np.abs(x2))
    bound1 = (2 * U_BF16 + U_BF16 ** 2) * (1 + U_BF16) * terms + U_BF16 * np.abs(exact1) + noise
    bound2 = (2 * U_BF16 + U_BF16 ** 2) * (1 + U_BF16) * cross + U_BF16 * np.abs(exact2) + noise
    assert np.all(np.abs(got[:, :, d1] - exact1) <= bound1)
    assert np.all(np.abs(got[:, :, d2] - exact2) <= bound2)
    # ...and it is a different result from the fused single rounding.
    fused = ko.rerotate_rows_c(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.F32,
                               rotary_dim=128, neox=True, prefix=0)
    assert (fused != eager).mean() > 0.1


@pytest.mark.parametrize("key_dtype", [ko.BF16, ko.F16])
@pytest.mark.parametrize("cache_dtype", [ko.F32, ko.BF16, ko.F16])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rotary_dim,prefix", [(64, 0), (32, 17)])
def test_eager_restatements_equal_torch(key_dtype, cache_dtype, neox, rotary_dim, prefix):
    rows, local, global_, cache = _random_case(key_dtype=key_dtype, cache_dtype=cache_dtype, tokens=96,
                                               heads=3, head_dim=64, rotary_dim=rotary_dim)
    kwargs = dict(key_dtype=key_dtype, cache_dtype=cache_dtype, rotary_dim=rotary_dim, neox=neox,
                  prefix=prefix, rounding=ko.EAGER)
    want = _r1_bits(rows, local, global_, cache, key_dtype=key_dtype, cache_dtype=cache_dtype,
                    rotary_dim=rotary_dim, neox=neox, prefix=prefix)
    assert np.array_equal(ko.rerotate_rows_c(rows, local, global_, cache, **kwargs), want)
    assert np.array_equal(ko.rerotate_rows_numpy(rows, local, global_, cache, **kwargs), want)


# ---------------------------------------------------------------------------
# Fused rounding, bf16 K with a 16-bit table.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rotary_dim,prefix", [(128, 0), (64, 9)])
def test_fused_bf16_table_chain_is_torch_bf16_arithmetic(neox, rotary_dim, prefix):
    rows, local, global_, cache = _random_case(key_dtype=ko.BF16, cache_dtype=ko.BF16, rotary_dim=rotary_dim)
    fused = ko.rerotate_rows_c(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.BF16,
                               rotary_dim=rotary_dim, neox=neox, prefix=prefix)
    torch_bf16 = _r1_bits(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.BF16,
                          rotary_dim=rotary_dim, neox=neox, prefix=prefix)
    assert np.array_equal(fused, torch_bf16)


def _torch_mixed_chain(rows, local, global_, f16_cache, rotary_dim):
    """bf16 K with an fp16 table, evaluated with torch tensors: the table entries
    widened to fp32, each product cast to bf16, then bf16 sums and products."""

    half = rotary_dim // 2
    table = _torch_tensor(f16_cache, ko.F16).float()
    lc, ls = table[local, :half][:, None, :], table[local, half:rotary_dim][:, None, :]
    gc, gs = table[global_, :half][:, None, :], table[global_, half:rotary_dim][:, None, :]
    bf16 = torch.bfloat16
    dc = (gc * lc).to(bf16) + (gs * ls).to(bf16)
    ds = (gs * lc).to(bf16) - (gc * ls).to(bf16)
    key = _torch_tensor(rows, ko.BF16)
    x1, x2 = key[..., :half], key[..., half:rotary_dim]
    out = torch.cat((x1 * dc - x2 * ds, x2 * dc + x1 * ds, key[..., rotary_dim:]), dim=-1)
    return _bits(out)


def test_fused_f16_table_chain_is_torch_mixed_arithmetic():
    rows, local, global_, cache = _random_case(key_dtype=ko.BF16, cache_dtype=ko.F16)
    fused = ko.rerotate_rows_c(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.F16,
                               rotary_dim=128, neox=True, prefix=0)
    assert np.array_equal(fused, _torch_mixed_chain(rows, local, global_, cache, 128))


def _chain_geometry_excess(rerotate, *, cache_dtype, neox, table_override=None, rotary_dim=128,
                           tokens=512, heads=4, theta=1e6, max_position=2048) -> float:
    """Max over elements of |re-rotated - direct fp64 rotation| minus the derived
    bound, for bf16 keys and a 16-bit table (> 0: the bound is broken)."""

    rng = np.random.default_rng(SEED + 7)
    raw = rng.standard_normal((tokens, heads, rotary_dim))
    local = rng.integers(0, max_position, size=tokens)
    global_ = rng.integers(0, max_position, size=tokens)
    table = build_cos_sin_cache(max_position, rotary_dim, theta=theta).numpy()
    if table_override is not None:
        table = table_override(table)
    cache = ko.f32_to_bf16_bits(table) if cache_dtype == ko.BF16 else ko.f32_to_f16_bits(table)
    rows = ko.f32_to_bf16_bits(rope_math.rotate(raw, local, rotary_dim, theta=theta, neox=neox).astype(np.float32))
    out = rerotate(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=cache_dtype,
                   rotary_dim=rotary_dim, neox=neox, prefix=0)
    got = ko.bf16_bits_to_f32(out).astype(np.float64)
    want = rope_math.rotate(raw, global_, rotary_dim, theta=theta, neox=neox)
    d1, d2 = rope_math.pair_dims(rotary_dim, neox)
    # Table entries off by u_T each, products and the delta's sum rounded to
    # bf16: |dc - cos| <= 2 u_T + 2 u (likewise ds).  Rotation: both products
    # and the sum rounded (2 u), the key itself rounded to bf16 (u).  Scale:
    # |x1| + |x2| <= sqrt(2) times the pair's norm, which rotation preserves.
    # fp32 angles of positions < 2048 add < 2048 * 2^-23 relative.
    u_table = U_BF16 if cache_dtype == ko.BF16 else U_F16
    norm = np.sqrt(raw[:, :, d1] ** 2 + raw[:, :, d2] ** 2)
    bound = (np.sqrt(2) * norm * (2 * u_table + 5 * U_BF16) * 1.01 + norm * max_position * 2.0 ** -23 + 1e-6)
    error = np.maximum(np.abs(got[:, :, d1] - want[:, :, d1]), np.abs(got[:, :, d2] - want[:, :, d2]))
    return float((error - bound).max())


@pytest.mark.parametrize("cache_dtype", [ko.BF16, ko.F16])
@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("rerotate", [ko.rerotate_rows_c, ko.rerotate_rows_numpy])
def test_fused_16bit_table_chain_matches_direct_rotation(cache_dtype, neox, rerotate):
    assert _chain_geometry_excess(rerotate, cache_dtype=cache_dtype, neox=neox) <= 0.0


def test_chain_checks_catch_planted_mistakes():
    def swapped_direction(rows, local, global_, cache, **kw):
        return ko.rerotate_rows_numpy(rows, global_, local, cache, **kw)

    def wrong_pairing(rows, local, global_, cache, **kw):
        kw["neox"] = not kw["neox"]
        return ko.rerotate_rows_numpy(rows, local, global_, cache, **kw)

    def flipped_sign(table):
        table = table.copy()
        table[:, table.shape[1] // 2:] *= -1
        return table

    for cache_dtype in (ko.BF16, ko.F16):
        assert _chain_geometry_excess(swapped_direction, cache_dtype=cache_dtype, neox=True) > 0.1
        assert _chain_geometry_excess(wrong_pairing, cache_dtype=cache_dtype, neox=True) > 0.1
        assert _chain_geometry_excess(ko.rerotate_rows_numpy, cache_dtype=cache_dtype, neox=True,
                                      table_override=flipped_sign) > 0.1
    # Dropped roundings (products and sums kept in fp32: the widened table
    # through the fp32 path) keep the geometry but break the torch equality.
    rows, local, global_, cache = _random_case(key_dtype=ko.BF16, cache_dtype=ko.BF16)
    unrounded = ko.rerotate_rows_c(rows, local, global_, ko.bf16_bits_to_f32(cache), key_dtype=ko.BF16,
                                   cache_dtype=ko.F32, rotary_dim=128, neox=True, prefix=0)
    torch_bf16 = _r1_bits(rows, local, global_, cache, key_dtype=ko.BF16, cache_dtype=ko.BF16,
                          rotary_dim=128, neox=True)
    assert (unrounded != torch_bf16).mean() > 0.05
    rows, local, global_, cache = _random_case(key_dtype=ko.BF16, cache_dtype=ko.F16)
    unrounded = ko.rerotate_rows_c(rows, local, global_, ko.f16_bits_to_f32(cache), key_dtype=ko.BF16,
                                   cache_dtype=ko.F32, rotary_dim=128, neox=True, prefix=0)
    assert (unrounded != _torch_mixed_chain(rows, local, global_, cache, 128)).mean() > 0.05


# ---------------------------------------------------------------------------
# Fused rounding, fp16 K.
# ---------------------------------------------------------------------------
def _fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """fp32 fused multiply-add: a*b + c with one rounding (the fp32 product is
    exact in fp64; the fp64 sum's own rounding is far below fp32's)."""

    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def test_fp16_key_fused_branch_rounds_once_and_contraction_moves_it_at_most_one_ulp():
    rows, local, global_, cache = _random_case(key_dtype=ko.F16, cache_dtype=ko.F32, tokens=512)
    out = ko.rerotate_rows_c(rows, local, global_, cache, key_dtype=ko.F16, cache_dtype=ko.F32,
                             rotary_dim=128, neox=True, prefix=0)
    x1, x2, dc64, ds64, exact1, exact2, (d1, d2) = _exact_from_table(rows, local, global_, cache,
                                                                     key_dtype=ko.F16, cache_dtype=ko.F32)
    got = ko.f16_bits_to_f32(out).astype(np.float64)
    noise = 8 * 2.0 ** -24 * (np.abs(x1) + np.abs(x2))
    assert np.all(np.abs(got[:, :, d1] - exact1) <= 0.5 * rope_math.f16_ulp(exact1) + noise)
    assert np.all(np.abs(got[:, :, d2] - exact2) <= 0.5 * rope_math.f16_ulp(exact2) + noise)

    # The same rotation with every multiply-add contracted (delta and rotation).
    half = 64
    lc, ls = cache[local, :half][:, None, :], cache[local, half:][:, None, :]
    gc, gs = cache[global_, :half][:, None, :], cache[global_, half:][:, None, :]
    dc = _fma32(gc, lc, gs * ls)
    ds = _fma32(gs, lc, -(gc * ls))
    a1, a2 = x1.astype(np.float32), x2.astype(np.float32)
    o1 = ko.f32_to_f16_bits(_fma32(a1, dc, -(a2 * ds)))
    o2 = ko.f32_to_f16_bits(_fma32(a2, dc, a1 * ds))
    contracted = np.stack([ko.f16_bits_to_f32(o1), ko.f16_bits_to_f32(o2)]).astype(np.float64)
    ours = np.stack([got[:, :, d1], got[:, :, d2]])
    assert np.all(np.abs(contracted - ours) <= rope_math.f16_ulp(ours))
