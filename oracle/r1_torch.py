"""Torch restatement of the reference's eager batched link path (rounding "R1").

TEST INFRASTRUCTURE ONLY: used by tests/ to report how far the fused
semantics are from the eager torch path, and by bench.py as the CPU baseline
(timed on the host cores).  Never part of the product path.

Follows, in order:
* patched_sglang_files/python/sglang/srt/pic_runtime.py:5534-5599
  per layer: K = K_l.index_select(0, src), V = V_l.index_select(0, src);
  K[prefix:] = remap(K[prefix:]); K = cat(K[:prefix], remapped);
  K_l.index_copy_(0, dst, K); V_l.index_copy_(0, dst, V)
* pic_runtime.py:6025-6058 (_remap_key_positions)
  lc, ls = cache.index_select(0, local).chunk(2, -1); gc, gs likewise;
  delta_cos = gc*lc + gs*ls; delta_sin = gs*lc - gc*ls (fp32)
* pic_runtime.py:1868-1885 (_apply_rotary_emb)
  cos, sin cast to the key dtype; out1 = x1*cos - x2*sin, out2 = x2*cos + x1*sin,
  each op rounded to the key dtype; neox halves or GPT-J interleave.

The eager path copies repair rows too (they are overwritten by the repair
pass afterwards); it has no repair mask.
"""

from __future__ import annotations

import torch


def apply_rotary_emb(
    x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, is_neox_style: bool
) -> torch.Tensor:
    cos = cos.unsqueeze(-2).to(x.dtype)
    sin = sin.unsqueeze(-2).to(x.dtype)
    if is_neox_style:
        x1, x2 = torch.chunk(x, 2, dim=-1)
    else:
        x1 = x[..., ::2]
        x2 = x[..., 1::2]
    out1 = x1 * cos - x2 * sin
    out2 = x2 * cos + x1 * sin
    if is_neox_style:
        return torch.cat((out1, out2), dim=-1)
    return torch.stack((out1, out2), dim=-1).flatten(-2)


def remap_key_positions(
    key: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    rotary_dim: int,
    is_neox_style: bool,
) -> torch.Tensor:
    """key [n, H, D] rotated from local to global positions (R1)."""

    cache = cos_sin_cache[:, :rotary_dim]
    local_cos, local_sin = cache.index_select(0, local_positions).chunk(2, dim=-1)
    global_cos, global_sin = cache.index_select(0, global_positions).chunk(2, dim=-1)
    key_rot = key[..., :rotary_dim]
    key_pass = key[..., rotary_dim:]
    delta_cos = global_cos * local_cos + global_sin * local_sin
    delta_sin = global_sin * local_cos - global_cos * local_sin
    rerotated = apply_rotary_emb(key_rot, delta_cos, delta_sin, is_neox_style)
    return torch.cat((rerotated, key_pass), dim=-1)


def link_batched_layers(
    key_layers: list[torch.Tensor],
    value_layers: list[torch.Tensor],
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
    local_positions: torch.Tensor,
    global_positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    *,
    prefix_token_count: int,
    rotary_dim: int,
    is_neox_style: bool,
) -> None:
    """In-place eager link of every layer, as the reference's torch branch does."""

    tail = int(source_slots.numel()) - int(prefix_token_count)
    for key_buffer, value_buffer in zip(key_layers, value_layers):
        key = key_buffer.index_select(0, source_slots)
        value = value_buffer.index_select(0, source_slots)
        if tail:
            remapped = remap_key_positions(
                key[prefix_token_count:],
                local_positions[prefix_token_count:],
                global_positions[prefix_token_count:],
                cos_sin_cache,
                rotary_dim,
                is_neox_style,
            )
            key = torch.cat((key[:prefix_token_count], remapped))
        key_buffer.index_copy_(0, destination_slots, key)
        value_buffer.index_copy_(0, destination_slots, value)


def scatter_rows(
    key_layers: list[torch.Tensor],
    value_layers: list[torch.Tensor],
    destination_slots: torch.Tensor,
    repaired_keys: torch.Tensor,
    repaired_values: torch.Tensor,
) -> None:
    """The repair pass's write-back (flashinfer_sparse_repair.py:2235-2239)."""

    for layer, (key_buffer, value_buffer) in enumerate(zip(key_layers, value_layers)):
        key_buffer.index_copy_(0, destination_slots, repaired_keys[layer])
        value_buffer.index_copy_(0, destination_slots, repaired_values[layer])
