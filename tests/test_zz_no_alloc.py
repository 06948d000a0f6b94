"""The allocation-free attention entry point (ca_attn_fwd_noalloc), called through the C-ABI,
against ca_attn_fwd with a caller workspace: two calls in a row on one GPU (the second with a
smaller input, after the first left its partials in the library's scratch array), each bit
for bit equal to ca_attn_fwd at the same split count; num_splits = 0 equal to ca_attn_fwd's
num_splits = 0 when the automatic count fits the array, and to the lowered fixed count when it
does not (a ragged batch whose two automatic splits need 56 MiB); a split count whose partials
exceed the array refused on the host."""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

from compactattention_amd import _hip, ops
from compactattention_amd.synthetic import make_chunk, make_chunk_device

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(128)


def _tables(ch, hkv, cap, topk=4):
    P = ch.past_blocks
    kmean = torch.zeros((hkv, cap, 128), dtype=torch.float32, device=ch.q.device)
    ops.cache_fill(ch.k[:, :, :cap * 64].transpose(1, 2).contiguous(), None, None, None, [0], cap, kmean)
    qhat = ops.pool_query(ch.q, P, cap)
    rowmask, _ = ops.score_select(qhat, kmean, SCALE, ops.Rule(topk=topk, sink_blocks=1, local_blocks=2), P, hkv,
                                  cap)
    return ops.union_compact(rowmask, P, hkv, cap)[:2]


def _noalloc(q, K, V, table, counts, P, cap, hkv, out, lse, num_splits):
    d = ops.make_dims(q.shape[0], q.shape[1], q.shape[2], hkv, cap)
    ql, ol = ops.seq_layout(q, "q"), ops.seq_layout(out, "out")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return _hip.lib().ca_attn_fwd_noalloc(ctypes.byref(d), ctypes.byref(ql), ctypes.byref(K.layout),
                                          ctypes.byref(V.layout), table.data_ptr(), table.stride(0),
                                          counts.data_ptr(), ops.past_array(P), SCALE, ctypes.byref(ol),
                                          lse.data_ptr(), int(num_splits), stream)


def _check_equal(ch, K, V, table, counts, cap, hkv, num_splits, ref_splits, gpu):
    B, lq, hq = ch.q.shape[:3]
    P = ch.past_blocks
    ref, ref_lse = ops.attn_fwd(ch.q, K, V, table, counts, P, SCALE, cap, hkv, with_lse=True,
                                num_splits=ref_splits)
    out = torch.full_like(ch.q, float("nan"))
    lse = torch.full((B, hq, lq), float("nan"), device=gpu)
    rc = _noalloc(ch.q, K, V, table, counts, P, cap, hkv, out, lse, num_splits)
    assert rc == _hip.CA_OK, _hip.last_error()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (num_splits, ref_splits)
    assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32)), (num_splits, ref_splits)
    return out, lse


def test_noalloc_matches_workspace_entry(gpu):
    for past, lq, hq, hkv in ((32768, 1024, 32, 8), (8192, 256, 8, 2)):  # the second call is smaller
        print(f"case: noalloc past={past} chunk={lq} heads={hq}/{hkv}", flush=True)
        ch = make_chunk_device(past, lq, hq, hkv, gpu, seed=past)
        cap, P = ch.kv_cap, ch.past_blocks
        table, counts = _tables(ch, hkv, cap)
        K, V = ops.KV.heads_first(ch.k), ops.KV.heads_first(ch.v)
        splits = ops.attn_pick_splits(P, lq, hq, hkv, cap)
        if past == 32768:
            assert splits > 1  # the first call runs through the scratch array
            # a forced split count whose partials exceed the array (16 splits: ~270 MB): refused on the host
            assert ops.attn_workspace_bytes(P, lq, hq, hkv, cap, 16) > _hip.STATIC_SCRATCH_BYTES
            out = torch.empty_like(ch.q)
            lse = torch.empty((1, hq, lq), device=gpu)
            rc = _noalloc(ch.q, K, V, table, counts, P, cap, hkv, out, lse, 16)
            assert rc == _hip.CA_ERR_LIMIT and "CA_STATIC_SCRATCH_BYTES" in _hip.last_error()
        assert ops.attn_workspace_bytes(P, lq, hq, hkv, cap, splits) <= _hip.STATIC_SCRATCH_BYTES
        _check_equal(ch, K, V, table, counts, cap, hkv, 0, 0, gpu)       # the automatic plan, as ca_attn_fwd(0)
        _check_equal(ch, K, V, table, counts, cap, hkv, splits, splits, gpu)


def test_noalloc_lowers_an_automatic_count_that_does_not_fit(gpu):
    """A ragged batch (BASELINE config 4's heads and chunk, shorter pasts): ca_attn_fwd's automatic
    count is 2 splits, whose partials (56 MiB) exceed the array; num_splits = 0 lowers it to 1
    and equals ca_attn_fwd with one split bit for bit."""
    past_tokens, lq, hq, hkv = [1024, 3072, 6144, 8192], 512, 28, 4
    print(f"case: noalloc ragged past={past_tokens} chunk={lq} heads={hq}/{hkv}", flush=True)
    ch = make_chunk(past_tokens, lq, hq, hkv, seed=77)
    ch.q, ch.k, ch.v = ch.q.to(gpu), ch.k.to(gpu), ch.v.to(gpu)
    cap, P = ch.kv_cap, ch.past_blocks
    auto = ops.attn_pick_splits(P, lq, hq, hkv, cap)
    assert auto == 2 and ops.attn_workspace_bytes(P, lq, hq, hkv, cap, auto) > _hip.STATIC_SCRATCH_BYTES
    kmean = torch.zeros((len(P) * hkv, cap, 128), dtype=torch.float32, device=gpu)
    ops.cache_fill(ch.k.transpose(1, 2).contiguous(), None, None, None, [0] * len(P), cap, kmean)
    qhat = ops.pool_query(ch.q, P, cap)
    rowmask, _ = ops.score_select(qhat, kmean, SCALE, ops.Rule(topk=8, sink_blocks=1, local_blocks=2), P, hkv, cap)
    table, counts = ops.union_compact(rowmask, P, hkv, cap)[:2]
    K, V = ops.KV.heads_first(ch.k), ops.KV.heads_first(ch.v)
    _check_equal(ch, K, V, table, counts, cap, hkv, 0, 1, gpu)
