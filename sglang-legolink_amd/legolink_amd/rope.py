"""RoPE cos/sin table in the layout the link operator reads.

Row p holds ``cos(p * inv_freq)`` in columns ``[0, rotary_dim/2)`` and
``sin(p * inv_freq)`` in ``[rotary_dim/2, rotary_dim)``, with
``inv_freq = 1 / theta ** (arange(0, rotary_dim, 2) / rotary_dim)``, all fp32.
This is the recipe the reference's fixtures use (tests/pic/support.py:57-71,
tests/test_sglang_pic_runtime.py:73-86) for the rotary module's
``cos_sin_cache``; Qwen2.5 / Qwen3 use theta = 1e6 and rotary_dim = head_dim
(patched_sglang_files/python/sglang/srt/models/qwen2.py:110-177).

The table is built once per model on the host, like the rotary module's own
cache, and then moved to the device.  It is an input of the link, not part of
the link's computation.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional

import torch

QWEN_ROPE_THETA = 1_000_000.0


def build_cos_sin_cache(
    max_positions: int,
    rotary_dim: int,
    *,
    theta: float = QWEN_ROPE_THETA,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    if rotary_dim <= 0 or rotary_dim % 2:
        raise ValueError("rotary_dim must be positive and even")
    inv_freq = 1.0 / (
        theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim)
    )
    positions = torch.arange(int(max_positions), dtype=torch.float32)
    angles = torch.outer(positions, inv_freq)
    return torch.cat((angles.cos(), angles.sin()), dim=-1).to(dtype)


@dataclass
class RotarySpec:
    """What the link needs of a layer's rotary embedding.

    A link whose positions run past the end of ``cos_sin_cache`` grows it
    before launching (patched_sglang_files/python/sglang/srt/
    pic_runtime.py:5051-5053, :6040).  How depends on where the table came
    from:

    * ``module``: the model's rotary module (anything with ``cos_sin_cache``
      and ``_ensure_cos_sin_cache_length``, as sglang's rotary embeddings
      have).  Growth is delegated to it, so the model's own scaling (YaRN,
      llama3, linear, ...) is kept, and the grown table is read back from it.
    * ``theta``: the table is the plain-theta table of ``build_cos_sin_cache``.
      It is rebuilt longer from theta, and the rebuild must reproduce every
      existing row bit for bit, or the growth raises (the table was not that
      recipe).
    * neither: a table that is too short raises ``ValueError``.
    """

    cos_sin_cache: torch.Tensor
    rotary_dim: int
    is_neox_style: bool = True
    theta: Optional[float] = None
    module: Any = None

    @classmethod
    def from_module(cls, module: Any) -> "RotarySpec":
        """Wrap a model's rotary module (``cos_sin_cache``, ``rotary_dim``,
        ``is_neox_style``); the table is grown through the module."""

        for name in ("cos_sin_cache", "rotary_dim"):
            if not hasattr(module, name):
                raise ValueError(f"rotary module has no {name}")
        return cls(module.cos_sin_cache, int(module.rotary_dim),
                   is_neox_style=bool(getattr(module, "is_neox_style", True)), module=module)

    @classmethod
    def for_theta(cls, max_positions: int, rotary_dim: int, *, theta: float = QWEN_ROPE_THETA,
                  is_neox_style: bool = True) -> "RotarySpec":
        """A plain-theta table that can grow itself."""

        return cls(build_cos_sin_cache(max_positions, rotary_dim, theta=theta), rotary_dim,
                   is_neox_style=is_neox_style, theta=theta)

    def ensure_cos_sin_cache_length(self, needed_max_position: int) -> None:
        """Make row ``needed_max_position`` of the table exist."""

        needed = int(needed_max_position)
        rows = int(self.cos_sin_cache.shape[0])
        if needed < rows:
            return
        if self.module is not None:
            self.module._ensure_cos_sin_cache_length(needed)
            table = self.module.cos_sin_cache
            if int(table.shape[0]) <= needed:
                raise ValueError(f"the rotary module's table has {int(table.shape[0])} rows after growing it "
                                 f"to position {needed}")
            self.cos_sin_cache = table
            return
        if self.theta is None:
            raise ValueError(f"cos/sin table has {rows} rows, position {needed} is needed, and the table "
                             "cannot grow: give RotarySpec the model's rotary module or the theta it was "
                             "built with")
        grown = build_cos_sin_cache(max(needed + 1, 2 * rows), self.rotary_dim, theta=self.theta,
                                    dtype=self.cos_sin_cache.dtype).to(self.cos_sin_cache.device)
        if not torch.equal(grown[:rows], self.cos_sin_cache):
            raise ValueError(f"cos/sin table is not the theta={self.theta:g} table of rotary_dim "
                             f"{self.rotary_dim}; it cannot be grown from theta")
        self.cos_sin_cache = grown
