"""CPU oracle of the sparse repair attention.

TEST INFRASTRUCTURE ONLY: only tests/ may import this module, to check the
repair attention kernel.  The product path never calls it.

Restates, in float64 numpy:

* ``logical_causal_mask`` -- key position j is visible to query position p
  iff j <= p (tests/pic/reference/attention_reference.py:8-12);
* ``gqa_attention`` -- per query and query head h, softmax over the visible
  keys of scale * q . k (scale 1 / sqrt(head_dim) by default) times V, reading
  KV head h // (num_q_heads // num_kv_heads) (attention_reference.py:14-48);
* ``repair_attention`` -- the physical-slot form the reference builds in
  ``build_explicit_causal_masked_pattern``
  (patched_sglang_files/python/sglang/srt/flashinfer_sparse_repair.py:1241-1263):
  keys and values of a repair span [start, end) are the pool rows at
  slot_ids[0:end], in logical order, with the logical causal mask of query
  positions start..end-1.  Slots outside the pool are invisible keys.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np


def logical_causal_mask(query_positions: np.ndarray, kv_positions: np.ndarray) -> np.ndarray:
    return np.asarray(kv_positions)[None, :] <= np.asarray(query_positions)[:, None]


def gqa_attention(query: np.ndarray, key: np.ndarray, value: np.ndarray, visible: np.ndarray, *,
                  scale: Optional[float] = None) -> np.ndarray:
    """query [q, hq, d], key/value [kv, hkv, d], visible bool [q, kv] -> float64 [q, hq, d]."""

    query = np.asarray(query, dtype=np.float64)
    key = np.asarray(key, dtype=np.float64)
    value = np.asarray(value, dtype=np.float64)
    q_tokens, q_heads, head_dim = query.shape
    kv_tokens, kv_heads, _ = value.shape
    if key.shape != (kv_tokens, kv_heads, head_dim) or visible.shape != (q_tokens, kv_tokens):
        raise ValueError("shape mismatch")
    if q_heads % kv_heads:
        raise ValueError("query heads must be divisible by KV heads")
    group = q_heads // kv_heads
    factor = scale if scale is not None else 1.0 / math.sqrt(head_dim)
    out = np.zeros((q_tokens, q_heads, value.shape[2]), dtype=np.float64)
    for h in range(q_heads):
        kv = h // group
        scores = (query[:, h, :] @ key[:, kv, :].T) * factor          # [q, kv]
        scores = np.where(visible, scores, -np.inf)
        top = scores.max(axis=1, keepdims=True)
        top = np.where(np.isfinite(top), top, 0.0)
        weights = np.exp(scores - top)
        total = weights.sum(axis=1, keepdims=True)
        out[:, h, :] = (weights @ value[:, kv, :]) / np.where(total > 0, total, 1.0)
    return out


def repair_attention(query: np.ndarray, key_pool: np.ndarray, value_pool: np.ndarray,
                     slot_ids: Sequence[int], repair_start: int, repair_end: int, *,
                     scale: Optional[float] = None) -> np.ndarray:
    """One repair span: query [end - start, hq, d]; pools [slots, hkv, d]."""

    slots = np.asarray(slot_ids, dtype=np.int64)[:repair_end]
    valid = (slots >= 0) & (slots < key_pool.shape[0])
    safe = np.where(valid, slots, 0)
    visible = logical_causal_mask(np.arange(repair_start, repair_end), np.arange(repair_end)) & valid[None, :]
    # An invalid slot contributes nothing, whatever the pool holds at the row it
    # would alias: its K and V rows are zeros (an invisible key with a NaN value
    # would otherwise leak through 0 * NaN).
    keys = np.where(valid[:, None, None], np.asarray(key_pool)[safe], 0.0)
    values = np.where(valid[:, None, None], np.asarray(value_pool)[safe], 0.0)
    return gqa_attention(query, keys, values, visible, scale=scale)
