"""Sparse repair attention: the repair pass's attention over the linked KV.

After a link, the repair pass recomputes the ``imp_indices`` rows. Each
contiguous repair span [repair_start, repair_end) of a request attends over the
request's tokens at logical positions 0 .. repair_end - 1, which live in
physical pool slots, under the explicit logical causal rule: query position p
sees exactly the positions j <= p.  The reference runs this as a FlashInfer
block-sparse attention over physical slot ids with that rule carried in a
mask (patched_sglang_files/python/sglang/srt/flashinfer_sparse_repair.py:
``build_explicit_causal_masked_pattern`` :1241-1263, the plan/run of
``_try_flashinfer_sparse_attention_single`` :2009-2272, the row batching of
``build_grouped_explicit_causal_masked_pattern`` :1266-1318), and restates its
semantics as ``gqa_attention`` over ``logical_causal_mask``
(tests/pic/reference/attention_reference.py:8-48).

Here it is one hand-written gfx950 kernel (fp16 or bf16 MFMA, online softmax in fp32)
behind ``ll_repair_attention``, with the same two phases as the reference's
wrapper: a host plan built once per request batch (shared by every layer:
the slots and spans do not depend on the layer) and a run per layer.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

from . import _host_sequences, _native


class SparseRepairAttentionError(RuntimeError):
    """A repair attention request that must not run (flashinfer_sparse_repair.py:65-66)."""


def _int64_values(values: Sequence) -> np.ndarray:
    """Span bounds as int64: integers read in C, anything else through int()."""

    out = np.empty(len(values), dtype=np.int64)
    try:
        _host_sequences.int64_from_sequence(values, out)
    except (TypeError, OverflowError):
        out = np.array([int(value) for value in values], dtype=np.int64)
    return out


class RepairAttentionPlan:
    """The work of one repair batch: ``spans`` is a list of
    ``(slot_ids, repair_start, repair_end)`` in query order -- the queries of
    span i are the next ``repair_end - repair_start`` rows of the query tensor.
    ``slot_ids[j]`` is the pool slot of logical position j of that span's
    request; spans of one request share its slot tensor.

    With ``validate`` (the reference always checks, :1235-1236) every slot of
    every span is checked against ``pool_size`` once, here (one device sync);
    without it, slots outside the pool are treated as invisible keys.

    With ``allocation_free`` no workspace is allocated: ``run`` calls
    ``ll_repair_attention_noalloc``, whose split partials live in the
    library's device scratch array (plans that need more than it holds are
    rejected when they run; runs that overlap on one GPU race).
    """

    def __init__(self, spans: Sequence[tuple[torch.Tensor, int, int]], *, num_q_heads: int,
                 num_kv_heads: int, head_dim: int, pool_size: Optional[int] = None,
                 split_tokens: int = 0, validate: bool = True, allocation_free: bool = False) -> None:
        if not spans:
            raise SparseRepairAttentionError("no repair spans")
        self.num_q_heads = int(num_q_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        device = spans[0][0].device
        tensors, starts, ends = zip(*spans)
        starts, ends = _int64_values(starts), _int64_values(ends)
        # Spans of one request share its slot tensor: each distinct tensor is
        # checked once, each span's range every time (the checks and messages
        # of build_explicit_causal_pattern, :1217-1238), and the error raised
        # is the one the first failing span meets, tensor checks first.
        ids = list(map(id, tensors))
        # Distinct tensors in order of first use, and the span that first uses each.
        first_use = dict(zip(reversed(ids), range(len(ids) - 1, -1, -1)))
        first_spans = [first_use[key] for key in dict.fromkeys(ids)]
        distinct = [tensors[index] for index in first_spans]
        position_of = {ids[index]: position for position, index in enumerate(first_spans)}
        span_tensor = np.fromiter(map(position_of.__getitem__, ids), dtype=np.int64, count=len(ids))
        failures = []  # (span index, message)
        for index, slot_ids in zip(first_spans, distinct):
            if slot_ids.ndim != 1:
                failures.append((index, "slot_ids must be rank 1"))
            elif slot_ids.device != device:
                failures.append((index, "repair spans must share one device"))
            elif slot_ids.dtype not in (torch.int32, torch.int64):
                failures.append((index, "slot_ids must be int32 or int64"))
        lengths = np.fromiter((int(t.numel()) for t in distinct), dtype=np.int64, count=len(distinct))
        bad_range = np.flatnonzero((starts < 0) | (ends <= starts))
        if bad_range.size:
            failures.append((int(bad_range[0]), "invalid repair range"))
        short = np.flatnonzero(lengths[span_tensor] < ends)
        if short.size:
            failures.append((int(short[0]), "slot_ids is shorter than repair_end"))
        if failures:
            raise SparseRepairAttentionError(min(failures, key=lambda failure: failure[0])[1])
        tables = [t.contiguous() for t in distinct]
        bases = np.zeros(len(distinct), dtype=np.int64)
        np.cumsum(lengths[:-1], out=bases[1:])
        counts = ends - starts
        rows = np.empty((len(ids), 4), dtype=np.int64)
        rows[0, 0] = 0
        np.cumsum(counts[:-1], out=rows[1:, 0])
        rows[:, 1] = starts
        rows[:, 2] = counts
        rows[:, 3] = bases[span_tensor]
        self.num_queries = int(counts.sum())
        self.span_starts, self.span_ends = starts, ends
        dtype = distinct[0].dtype if all(t.dtype == distinct[0].dtype for t in distinct) else torch.int64
        table = tables[0] if len(tables) == 1 else torch.cat([t.to(dtype) for t in tables])
        if validate and pool_size is not None:
            # Each tensor's slots up to its spans' largest end are checked
            # once: the smallest and largest with one reduction.
            reach = np.zeros(len(distinct), dtype=np.int64)
            np.maximum.at(reach, span_tensor, ends)
            needed = [t[: int(r)] for t, r in zip(tables, reach.tolist())]
            needed = needed[0] if len(needed) == 1 else torch.cat([t.to(dtype) for t in needed])
            low, high = torch.aminmax(needed)
            if int(low) < 0 or int(high) >= int(pool_size):
                raise SparseRepairAttentionError("slot_ids contains invalid KV slots")
        self.kv_slots = table
        self.rows = rows
        items, combine, positions, info = _native.repair_attention_plan(rows, self.num_q_heads,
                                                                        self.num_kv_heads, split_tokens)
        self.info = {"num_items": int(info.num_items), "num_combine": int(info.num_combine),
                     "workspace_items": int(info.workspace_items), "split_tokens": int(info.split_tokens)}
        packed = np.concatenate((items.reshape(-1), combine.reshape(-1), positions)).astype(np.int32)
        self._tables = torch.from_numpy(packed).to(device)  # one copy to the device
        self.items = self._tables[: items.size]
        self.combine = self._tables[items.size : items.size + combine.size]
        self.positions = self._tables[items.size + combine.size :]
        per_item = self.num_q_heads * (8 * self.head_dim + 32)  # 16 x head_dim 16-bit values, 16 (m, l) pairs
        self.allocation_free = bool(allocation_free)
        self.workspace = (torch.empty(info.workspace_items * per_item, dtype=torch.float32, device=device)
                          if info.workspace_items and not self.allocation_free else None)

    @property
    def algorithmic_flops(self) -> int:
        """4 * head_dim flops per (query, visible key) pair and query head."""

        starts, ends = self.span_starts.tolist(), self.span_ends.tolist()
        pairs = sum((end - start) * (start + end + 1) // 2 for start, end in zip(starts, ends))
        return 4 * self.head_dim * self.num_q_heads * pairs

    @property
    def kv_bytes_read(self) -> int:
        """Bytes of K and V the kernel gathers: each work item reads its KV range
        [kv_begin, kv_end) once per KV head (2-byte elements).  A lower bound
        at head dim 256, where a work item's 16 (tile, head) pairs take two
        workgroups, each of which gathers the keys its own tiles need."""

        items = self.items.view(-1, _native.REPAIR_ITEM_INTS).cpu().numpy().astype(np.int64)
        tokens = int((items[:, 2] - items[:, 1]).sum())
        return tokens * self.num_kv_heads * self.head_dim * 2 * 2

    def run(self, query: torch.Tensor, key_buffer: torch.Tensor, value_buffer: torch.Tensor, *,
            scale: Optional[float] = None, output: Optional[torch.Tensor] = None,
            stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """One layer: ``query`` [num_queries, num_q_heads, head_dim] fp16 or bf16
        (or its [num_queries, num_q_heads * head_dim] view), ``key_buffer`` /
        ``value_buffer`` the layer's [slots, num_kv_heads, head_dim] pool buffers
        of the same dtype.  Returns (or fills) the [num_queries, num_q_heads,
        head_dim] output, in that dtype."""

        shape = (self.num_queries, self.num_q_heads, self.head_dim)
        query = query.view(shape)
        # The checks of the reference's _compatibility_error
        # (flashinfer_sparse_repair.py:973-980).
        if query.dtype not in (torch.float16, torch.bfloat16):
            raise SparseRepairAttentionError(f"unsupported Q dtype: {query.dtype}")
        if key_buffer.dtype != query.dtype or value_buffer.dtype != query.dtype:
            raise SparseRepairAttentionError("Q/K/V dtypes must match")
        for name, tensor in (("query", query), ("key_buffer", key_buffer), ("value_buffer", value_buffer)):
            if not tensor.is_cuda:
                raise SparseRepairAttentionError(f"{name} must be a device tensor")
            if not tensor.is_contiguous():
                raise SparseRepairAttentionError(f"{name} must be contiguous")
        if key_buffer.ndim != 3 or key_buffer.shape[1:] != (self.num_kv_heads, self.head_dim) or (
                value_buffer.shape != key_buffer.shape):
            raise SparseRepairAttentionError("KV buffers must be [slots, num_kv_heads, head_dim]")
        if output is None:
            output = torch.empty(shape, dtype=query.dtype, device=query.device)
        elif output.shape != shape or output.dtype != query.dtype or not output.is_contiguous():
            raise SparseRepairAttentionError("output must be a contiguous tensor of the query's shape and dtype")
        args = _native.RepairAttentionArgs()
        args.query = query.data_ptr()
        args.output = output.data_ptr()
        args.num_queries = self.num_queries
        args.key_buffer = key_buffer.data_ptr()
        args.value_buffer = value_buffer.data_ptr()
        args.num_slots = int(key_buffer.shape[0])
        args.num_q_heads = self.num_q_heads
        args.num_kv_heads = self.num_kv_heads
        args.head_dim = self.head_dim
        args.kv_dtype = _native.DTYPE_BFLOAT16 if query.dtype == torch.bfloat16 else _native.DTYPE_FLOAT16
        args.softmax_scale = float(scale) if scale is not None else 1.0 / math.sqrt(self.head_dim)
        args.kv_slots = self.kv_slots.data_ptr()
        args.kv_slots_dtype = _native.DTYPE_INT64 if self.kv_slots.dtype == torch.int64 else _native.DTYPE_INT32
        args.kv_slots_len = int(self.kv_slots.numel())
        args.items = self.items.data_ptr()
        args.num_items = self.info["num_items"]
        args.combine = self.combine.data_ptr() if self.info["num_combine"] else None
        args.num_combine = self.info["num_combine"]
        args.query_positions = self.positions.data_ptr()
        args.workspace = self.workspace.data_ptr() if self.workspace is not None else None
        args.workspace_items = self.info["workspace_items"]
        if stream is None:
            stream = torch.cuda.current_stream(query.device)
        if self.allocation_free:
            _native.repair_attention_noalloc(args, stream.cuda_stream)
        else:
            _native.repair_attention(args, stream.cuda_stream)
        return output


def sparse_repair_attention(query: torch.Tensor, key_buffer: torch.Tensor, value_buffer: torch.Tensor,
                            slot_ids: torch.Tensor, *, repair_start: int, repair_end: int,
                            scale: Optional[float] = None) -> torch.Tensor:
    """One repair span of one layer (the reference's single-row path):
    ``query`` [repair_end - repair_start, num_q_heads, head_dim]."""

    plan = RepairAttentionPlan([(slot_ids, repair_start, repair_end)], num_q_heads=int(query.shape[1]),
                               num_kv_heads=int(key_buffer.shape[1]), head_dim=int(key_buffer.shape[2]),
                               pool_size=int(key_buffer.shape[0]))
    return plan.run(query, key_buffer, value_buffer, scale=scale)


def _repair_ranges(metadata: dict) -> list[tuple[int, int]]:
    ranges = metadata.get("repair_ranges")
    if ranges:
        return [(int(r["start"]), int(r["end"])) for r in ranges]
    return [(int(metadata["repair_start"]), int(metadata["repair_end"]))]


def try_sparse_repair_attention(q: torch.Tensor, k: Optional[torch.Tensor], v: Optional[torch.Tensor], layer,
                                forward_batch, save_kv_cache: bool) -> Optional[torch.Tensor]:
    """The repair pass's attention at the reference's seam:
    ``try_flashinfer_sparse_attention(q, k, v, layer, forward_batch,
    save_kv_cache)`` (flashinfer_sparse_repair.py:1944-1972), which
    ``RadixAttention.forward`` calls for a batch that carries
    ``pic_sparse_repair_metadata`` (layers/radix_attention.py:125-135).

    Returns None -- the caller's native attention -- when the batch has no
    repair metadata or its metadata names the native backend
    (``actual_backend == "native"``, :2023-2024).  Otherwise:

    * the repair rows come from the metadata: ``repair_ranges`` (or
      ``repair_start`` / ``repair_end``); with several rows in a batch of
      several requests, row r is request ``req_pool_indices[r]``
      (_make_flashinfer_row_batch, :1516-1554), else every row is request
      ``req_pool_indices[0]``; a row's keys are that request's slots
      ``req_to_token[request, :end]`` (_physical_slot_identity, :1083-1087);
    * the plan is built at the first layer and kept in the metadata for the
      later ones (the reference keeps its planned wrapper there, :2193-2200);
    * with ``save_kv_cache`` the batch's new K/V are written to
      ``out_cache_loc`` through the pool's ``set_kv_buffer`` before the
      attention reads the pool (:2235-2239);
    * the output is ``[tokens, tp_q_head_num * head_dim]`` in q's dtype,
      with ``layer.scaling`` as the softmax scale.
    """

    metadata = getattr(forward_batch, "pic_sparse_repair_metadata", None)
    if not metadata or metadata.get("actual_backend") == "native":
        return None
    hq, hkv, dim = int(layer.tp_q_head_num), int(layer.tp_k_head_num), int(layer.head_dim)
    pool = forward_batch.token_to_kv_pool
    key_buffer = pool.get_key_buffer(layer.layer_id)
    value_buffer = pool.get_value_buffer(layer.layer_id)
    ranges = _repair_ranges(metadata)
    plan = metadata.get("_hip_repair_plan")
    plan_key = (str(key_buffer.device), int(key_buffer.shape[0]), hq, hkv, dim, tuple(ranges))
    if plan is None or metadata.get("_hip_repair_plan_key") != plan_key:
        requests = forward_batch.req_pool_indices
        batch_size = int(getattr(forward_batch, "batch_size", 1))
        per_row = len(ranges) > 1 and batch_size > 1
        if per_row and len(ranges) != batch_size:
            raise SparseRepairAttentionError("grouped repair rows must match the batch's requests")
        table = forward_batch.req_to_token_pool.req_to_token
        slots: dict[int, torch.Tensor] = {}
        spans = []
        for row, (start, end) in enumerate(ranges):
            request = int(requests[row if per_row else 0])
            if request not in slots:
                slots[request] = table[request].to(torch.int32)
            spans.append((slots[request], start, end))
        plan = RepairAttentionPlan(spans, num_q_heads=hq, num_kv_heads=hkv, head_dim=dim,
                                   pool_size=int(key_buffer.shape[0]))
        metadata["_hip_repair_plan"] = plan
        metadata["_hip_repair_plan_key"] = plan_key
    else:
        metadata["plan_reuse_calls"] = int(metadata.get("plan_reuse_calls", 0)) + 1
    if int(q.numel()) != plan.num_queries * hq * dim:
        raise SparseRepairAttentionError("query tokens do not match the repair rows")
    if save_kv_cache and k is not None:
        pool.set_kv_buffer(layer, forward_batch.out_cache_loc, k, v, getattr(layer, "k_scale", None),
                           getattr(layer, "v_scale", None))
    output = plan.run(q.reshape(plan.num_queries, hq, dim), key_buffer, value_buffer,
                      scale=float(getattr(layer, "scaling", 1.0 / math.sqrt(dim))))
    metadata["actual_backend"] = "hip_repair_attention"
    metadata["layer_calls"] = int(metadata.get("layer_calls", 0)) + 1
    metadata["run_calls"] = int(metadata.get("run_calls", 0)) + 1
    return output.view(-1, hq * dim)


# The reference's name for the seam, for callers written against it.
try_flashinfer_sparse_attention = try_sparse_repair_attention
