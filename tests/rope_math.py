"""Textbook RoPE in float64, independent of the link's delta formula.

Rotating by angle theta_i * p is done with cos/sin of the angle directly
(the reference keeps the same kind of explicit check in
tests/pic/reference/rope_reference.py:6-55); re-rotation l -> g is checked by
comparing with a direct rotation to g, never by composing the delta formula.
"""

from __future__ import annotations

import numpy as np


def inv_freq64(rotary_dim: int, theta: float) -> np.ndarray:
    return 1.0 / (theta ** (np.arange(0, rotary_dim, 2, dtype=np.float64) / rotary_dim))


def pair_dims(rotary_dim: int, neox: bool) -> tuple[np.ndarray, np.ndarray]:
    half = rotary_dim // 2
    if neox:
        first = np.arange(half)
        return first, first + half
    first = 2 * np.arange(half)
    return first, first + 1


def rotate(values: np.ndarray, positions: np.ndarray, rotary_dim: int, *, theta: float,
           neox: bool = True, angles: np.ndarray | None = None) -> np.ndarray:
    """values [T, H, D] float64 rotated to ``positions`` [T] (dims >= rotary_dim kept)."""

    values = np.asarray(values, dtype=np.float64)
    if angles is None:
        angles = np.asarray(positions, dtype=np.float64)[:, None] * inv_freq64(rotary_dim, theta)[None, :]
    cos = np.cos(angles)[:, None, :]
    sin = np.sin(angles)[:, None, :]
    d1, d2 = pair_dims(rotary_dim, neox)
    out = values.copy()
    x1 = values[:, :, d1]
    x2 = values[:, :, d2]
    out[:, :, d1] = x1 * cos - x2 * sin
    out[:, :, d2] = x2 * cos + x1 * sin
    return out


def fp32_table_angles(positions: np.ndarray, rotary_dim: int, theta: float) -> np.ndarray:
    """Angles exactly as an fp32 table computes them: fl32(fl32(p) * fl32(inv_freq))."""

    inv = (1.0 / (np.float32(theta) ** (np.arange(0, rotary_dim, 2, dtype=np.float32) / np.float32(rotary_dim)))).astype(np.float32)
    return (np.asarray(positions, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)


def bf16_ulp(values: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |values| (normal range)."""

    magnitude = np.maximum(np.abs(np.asarray(values, dtype=np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(magnitude)) - 7)


def f16_ulp(values: np.ndarray) -> np.ndarray:
    magnitude = np.maximum(np.abs(np.asarray(values, dtype=np.float64)), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(magnitude)) - 10)
