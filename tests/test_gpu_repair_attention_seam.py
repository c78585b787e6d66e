"""The repair attention at the reference's seam: try_flashinfer_sparse_attention(
q, k, v, layer, forward_batch, save_kv_cache) (flashinfer_sparse_repair.py:1944-1972),
driven as RadixAttention.forward drives it (layers/radix_attention.py:125-135)
with a forward batch shaped like the reference tests' fakes
(tests/test_sglang_pic_runtime.py:126, tests/pic/test_flashinfer_capacity.py:121-127):
repair metadata, req_pool_indices, req_to_token_pool, token_to_kv_pool and
out_cache_loc.  The output is checked against the fp64 oracle over the pool as
it stands after the batch's K/V write (the reference writes, then runs:
:2235-2239), within the attention tests' bound."""

from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from legolink_amd.link_runtime import KVPool
from legolink_amd.repair_attention import try_flashinfer_sparse_attention
from oracle import attention_oracle as ao
from tests.gpu_helpers import bits, report

pytestmark = pytest.mark.gpu

HQ, HKV, DIM, SLOTS, LAYERS = 28, 4, 128, 8192, 2


def _setup(device, seed):
    generator = torch.Generator(device=device).manual_seed(seed)
    pool = KVPool([torch.randn(SLOTS, HKV, DIM, generator=generator, device=device).to(torch.bfloat16)
                   for _ in range(LAYERS)],
                  [torch.randn(SLOTS, HKV, DIM, generator=generator, device=device).to(torch.bfloat16)
                   for _ in range(LAYERS)])
    # Request r's slots by logical position: a random permutation of the pool.
    table = torch.stack([torch.randperm(SLOTS, generator=generator, device=device)[:3000] for _ in range(6)])
    return generator, pool, table.to(torch.int32)


def _layer(layer_id):
    return SimpleNamespace(layer_id=layer_id, tp_q_head_num=HQ, tp_k_head_num=HKV, head_dim=DIM,
                           scaling=1.0 / math.sqrt(DIM), k_scale=None, v_scale=None)


def _check(output, query, pool, layer, table, rows):
    got = output.view(-1, HQ, DIM).float().cpu().numpy()
    q = query.view(-1, HQ, DIM).float().cpu().numpy()
    keys = pool.get_key_buffer(layer).float().cpu().numpy()
    values = pool.get_value_buffer(layer).float().cpu().numpy()
    cursor = 0
    for request, start, end in rows:
        n = end - start
        slots = table[request].cpu().numpy()
        want = ao.repair_attention(q[cursor : cursor + n], keys, values, slots, start, end, scale=1 / math.sqrt(DIM))
        size = ao.repair_attention(q[cursor : cursor + n], keys, np.abs(values), slots, start, end,
                                   scale=1 / math.sqrt(DIM))
        bound = 2.0 ** -7 * (size + np.abs(want)) + 1e-5
        assert (np.abs(got[cursor : cursor + n] - want) <= bound).all(), f"request {request} [{start}, {end})"
        cursor += n
    assert cursor == got.shape[0]


@pytest.mark.parametrize("save_kv_cache", [True, False])
def test_seam_writes_then_attends_one_request(gpu_device, save_kv_cache):
    report(f"seam: one request, save_kv_cache={save_kv_cache}")
    generator, pool, table = _setup(gpu_device, 11)
    start, end, request = 1200, 1232, 2
    metadata = {"requested_backend": "flashinfer", "actual_backend": "flashinfer_block_sparse",
                "repair_start": start, "repair_end": end}
    batch = SimpleNamespace(pic_sparse_repair_metadata=metadata, batch_size=1,
                            req_pool_indices=torch.tensor([request], device=gpu_device),
                            req_to_token_pool=SimpleNamespace(req_to_token=table), token_to_kv_pool=pool,
                            out_cache_loc=table[request, start:end].to(torch.int64))
    plans = []
    for layer in range(LAYERS):
        q = torch.randn(end - start, HQ * DIM, generator=generator, device=gpu_device).to(torch.bfloat16)
        k = torch.randn(end - start, HKV, DIM, generator=generator, device=gpu_device).to(torch.bfloat16)
        v = torch.randn(end - start, HKV, DIM, generator=generator, device=gpu_device).to(torch.bfloat16)
        before_k = bits(pool.get_key_buffer(layer)[batch.out_cache_loc])
        output = try_flashinfer_sparse_attention(q, k, v, _layer(layer), batch, save_kv_cache)
        torch.cuda.synchronize(gpu_device)
        assert output.shape == (end - start, HQ * DIM) and output.dtype == torch.bfloat16
        written_k = bits(pool.get_key_buffer(layer)[batch.out_cache_loc])
        written_v = bits(pool.get_value_buffer(layer)[batch.out_cache_loc])
        if save_kv_cache:
            assert np.array_equal(written_k, bits(k)) and np.array_equal(written_v, bits(v))
        else:
            assert np.array_equal(written_k, before_k)
        _check(output, q, pool, layer, table, [(request, start, end)])
        plans.append(metadata["_hip_repair_plan"])
    assert plans[0] is plans[1]  # planned once for every layer
    assert metadata["layer_calls"] == LAYERS and metadata["plan_reuse_calls"] == LAYERS - 1
    assert metadata["actual_backend"] == "hip_repair_attention"


def test_seam_grouped_rows_of_several_requests(gpu_device):
    """Several repair rows in a batch of several requests: row r is request
    req_pool_indices[r] (_make_flashinfer_row_batch, :1516-1554)."""

    report("seam: grouped rows")
    generator, pool, table = _setup(gpu_device, 12)
    rows = [(4, 300, 316), (1, 2500, 2516), (5, 17, 33)]
    metadata = {"requested_backend": "flashinfer", "actual_backend": "flashinfer_block_sparse",
                "repair_start": rows[0][1], "repair_end": rows[-1][2],
                "repair_ranges": [{"start": s, "end": e} for _, s, e in rows], "repair_row_count": len(rows)}
    loc = torch.cat([table[r, s:e] for r, s, e in rows]).to(torch.int64)
    batch = SimpleNamespace(pic_sparse_repair_metadata=metadata, batch_size=len(rows),
                            req_pool_indices=torch.tensor([r for r, _, _ in rows], device=gpu_device),
                            req_to_token_pool=SimpleNamespace(req_to_token=table), token_to_kv_pool=pool,
                            out_cache_loc=loc)
    tokens = sum(e - s for _, s, e in rows)
    q = torch.randn(tokens, HQ, DIM, generator=generator, device=gpu_device).to(torch.bfloat16)
    k = torch.randn(tokens, HKV * DIM, generator=generator, device=gpu_device).to(torch.bfloat16)
    v = torch.randn(tokens, HKV * DIM, generator=generator, device=gpu_device).to(torch.bfloat16)
    output = try_flashinfer_sparse_attention(q, k, v, _layer(1), batch, True)
    torch.cuda.synchronize(gpu_device)
    assert np.array_equal(bits(pool.get_key_buffer(1)[loc]).reshape(tokens, -1), bits(k))
    _check(output, q, pool, 1, table, rows)


def test_seam_declines_without_metadata_or_on_native(gpu_device):
    q = torch.zeros(4, HQ * DIM, dtype=torch.bfloat16, device=gpu_device)
    assert try_flashinfer_sparse_attention(q, None, None, _layer(0), SimpleNamespace(), True) is None
    batch = SimpleNamespace(pic_sparse_repair_metadata={"actual_backend": "native", "repair_start": 0,
                                                        "repair_end": 4})
    assert try_flashinfer_sparse_attention(q, None, None, _layer(0), batch, True) is None
