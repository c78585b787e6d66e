"""Growth of the cos/sin table when a link needs positions past its end.

The reference grows the model's own table through the rotary module
(patched_sglang_files/python/sglang/srt/pic_runtime.py:5051-5053, :6040), so
a scaled RoPE keeps its scaling.  RotarySpec delegates to the module when it
has one, rebuilds a plain-theta table only when the rebuild reproduces the
existing rows bit for bit, and otherwise refuses.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from legolink_amd.rope import RotarySpec, build_cos_sin_cache


def _closed_form(positions, rotary_dim, theta, scale=1.0):
    inv_freq = 1.0 / theta ** (np.arange(0, rotary_dim, 2, dtype=np.float64) / rotary_dim)
    angles = np.outer(np.asarray(positions, dtype=np.float64) / scale, inv_freq)
    return np.concatenate([np.cos(angles), np.sin(angles)], axis=-1)


class ScaledRotary:
    """A model rotary module with linear position scaling: row p holds the
    plain table's angles at p / scale, which no theta reproduces."""

    def __init__(self, rows, rotary_dim, theta, scale):
        self.rotary_dim, self.is_neox_style, self.theta, self.scale = rotary_dim, True, theta, scale
        self.grow_calls = []
        self.cos_sin_cache = self._table(rows)

    def _table(self, rows):
        inv_freq = 1.0 / self.theta ** (torch.arange(0, self.rotary_dim, 2, dtype=torch.float32) / self.rotary_dim)
        angles = torch.outer(torch.arange(rows, dtype=torch.float32) / self.scale, inv_freq)
        return torch.cat((angles.cos(), angles.sin()), dim=-1)

    def _ensure_cos_sin_cache_length(self, needed_max_pos):
        self.grow_calls.append(needed_max_pos)
        if needed_max_pos >= self.cos_sin_cache.shape[0]:
            self.cos_sin_cache = self._table(needed_max_pos + 1)


def test_theta_table_grows_and_keeps_its_rows():
    spec = RotarySpec.for_theta(64, 16, theta=1e4)
    before = spec.cos_sin_cache.clone()
    spec.ensure_cos_sin_cache_length(300)
    table = spec.cos_sin_cache
    assert table.shape[0] > 300 and table.dtype == torch.float32
    assert torch.equal(table[:64], before)
    # New rows follow the theta = 1e4 closed form (fp32 cos/sin of fp32 angles).
    np.testing.assert_allclose(table[64:301].numpy(), _closed_form(range(64, 301), 16, 1e4), atol=2e-4)
    # Already long enough: untouched.
    spec.ensure_cos_sin_cache_length(10)
    assert spec.cos_sin_cache is table


def test_growth_refuses_a_table_of_another_theta():
    spec = RotarySpec(build_cos_sin_cache(64, 16, theta=1e4), rotary_dim=16, theta=1e6)
    with pytest.raises(ValueError, match="not the theta"):
        spec.ensure_cos_sin_cache_length(100)
    assert spec.cos_sin_cache.shape[0] == 64


def test_growth_without_module_or_theta_raises():
    spec = RotarySpec(build_cos_sin_cache(32, 8, theta=5e5), rotary_dim=8)
    spec.ensure_cos_sin_cache_length(31)  # inside the table: fine
    with pytest.raises(ValueError, match="cannot grow"):
        spec.ensure_cos_sin_cache_length(32)


def test_growth_delegates_to_the_model_rotary_module():
    module = ScaledRotary(48, 16, theta=1e4, scale=4.0)
    spec = RotarySpec.from_module(module)
    before = spec.cos_sin_cache.clone()
    spec.ensure_cos_sin_cache_length(200)
    assert module.grow_calls == [200]
    assert spec.cos_sin_cache is module.cos_sin_cache and spec.cos_sin_cache.shape[0] == 201
    assert torch.equal(spec.cos_sin_cache[:48], before)
    # The scaling is kept: the plain theta table differs, the scaled closed form holds.
    np.testing.assert_allclose(spec.cos_sin_cache[48:].numpy(), _closed_form(range(48, 201), 16, 1e4, 4.0),
                               atol=2e-4)
    assert not torch.allclose(spec.cos_sin_cache[100:], build_cos_sin_cache(201, 16, theta=1e4)[100:])


def test_module_that_cannot_grow_raises():
    class Fixed(ScaledRotary):
        def _ensure_cos_sin_cache_length(self, needed_max_pos):
            if needed_max_pos >= self.cos_sin_cache.shape[0]:
                raise AssertionError("fixture RoPE cache is too short")

    spec = RotarySpec.from_module(Fixed(16, 8, theta=1e4, scale=1.0))
    with pytest.raises(AssertionError):
        spec.ensure_cos_sin_cache_length(16)

    class Lazy(ScaledRotary):
        def _ensure_cos_sin_cache_length(self, needed_max_pos):
            pass

    spec = RotarySpec.from_module(Lazy(16, 8, theta=1e4, scale=1.0))
    with pytest.raises(ValueError, match="after growing"):
        spec.ensure_cos_sin_cache_length(16)


def test_executor_wraps_a_rotary_module_once():
    from legolink_amd.link_runtime import KVLinkExecutor
    from legolink_amd.registry import LegoLinkBlockRegistry

    module = ScaledRotary(64, 16, theta=1e4, scale=2.0)
    executor = KVLinkExecutor(LegoLinkBlockRegistry(), module, end_layer=3)
    specs = {id(spec) for spec in executor.rotary_by_layer.values()}
    assert len(specs) == 1 and executor.rotary_by_layer[0].module is module
    other = ScaledRotary(64, 16, theta=1e4, scale=1.0)
    executor = KVLinkExecutor(LegoLinkBlockRegistry(), {0: module, 1: module, 2: other}, end_layer=3)
    assert executor.rotary_by_layer[0] is executor.rotary_by_layer[1]
    assert executor.rotary_by_layer[2].module is other
