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
    """What the link needs of a layer's rotary embedding."""

    cos_sin_cache: torch.Tensor
    rotary_dim: int
    is_neox_style: bool = True
    theta: float = QWEN_ROPE_THETA

    def ensure_cos_sin_cache_length(self, needed_max_position: int) -> None:
        """Grow the table so that row ``needed_max_position`` exists."""

        rows = int(self.cos_sin_cache.shape[0])
        if needed_max_position < rows:
            return
        grown = max(int(needed_max_position) + 1, 2 * rows)
        self.cos_sin_cache = build_cos_sin_cache(
            grown, self.rotary_dim, theta=self.theta, dtype=self.cos_sin_cache.dtype
        ).to(self.cos_sin_cache.device)
