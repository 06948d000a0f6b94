"""BASELINE configs at their full sizes on the GPU.  Config 2: a 131072-token paged heads-first
cache, a 1024-token chunk, 32 Q / 8 KV heads, FlashPrefill pooled top-k (k = 10) + sink block 0
+ 2 local blocks; config 1 (AttnGate at 32768 tokens) and config 4 (ragged batch) below.

The selection path is integer/fp32 work with a fixed evaluation order, so at this size it is
still checked bit for bit against the CPU oracle (which runs it in well under a second):
block means of the whole cache, pooled queries, per-row masks, the GQA union, tables and
counts.  The attention is checked on a sample of query tokens (the first and the last 8 of
the chunk, every head) against the fp64-accumulated oracle over the same selected blocks,
and through properties that hold at any size: the tables' structure, and agreement of the
automatic split plan with the unsplit launch.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from compactattention_amd import ops
from compactattention_amd.synthetic import make_chunk_device

from .util import bits, f32, float_bits_equal, unpack_rowmask

pytestmark = pytest.mark.gpu

PAST, LQ, HQ, HKV = 131072, 1024, 32, 8
TOPK = 10
ATOL_MAX = 2e-2
ATOL_MEAN = 2e-3


@pytest.fixture(scope="module")
def full(gpu):
    print("case: full-size config 2 (131072 past tokens, chunk 1024, 32/8 heads)", flush=True)
    ch = make_chunk_device(PAST, LQ, HQ, HKV, gpu)
    cap, P = ch.kv_cap, ch.past_blocks
    kc, vc = torch.zeros_like(ch.k), torch.zeros_like(ch.v)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((HKV, cap, 128), dtype=torch.float32, device=gpu)
    step = 16384
    for t0 in range(0, PAST, step):  # the past, then the chunk (the path's append)
        t1 = min(PAST, t0 + step)
        ops.cache_fill(ch.k[:, :, t0:t1].transpose(1, 2).contiguous(), ch.v[:, :, t0:t1].transpose(1, 2).contiguous(),
                       K, V, [t0 // 64], cap, kmean)
    ops.cache_fill(ch.k[:, :, PAST:PAST + LQ].transpose(1, 2).contiguous(),
                   ch.v[:, :, PAST:PAST + LQ].transpose(1, 2).contiguous(), K, V, P, cap, kmean)
    scale = 1.0 / math.sqrt(128)
    rule = ops.Rule(topk=TOPK, sink_blocks=1, local_blocks=2)
    qhat = ops.pool_query(ch.q, P, cap)
    rowmask, _ = ops.score_select(qhat, kmean, scale, rule, P, HKV, cap)
    table, counts, _, _ = ops.union_compact(rowmask, P, HKV, cap)
    torch.cuda.synchronize()
    return dict(ch=ch, cap=cap, P=P, K=K, V=V, kc=kc, vc=vc, kmean=kmean, qhat=qhat, rowmask=rowmask,
                table=table, counts=counts, scale=scale)


def test_fullsize_cache_and_selection_bit_exact(full):
    ch, cap, P = full["ch"], full["cap"], full["P"]
    nkb = P[0] + LQ // 64
    kbits = bits(ch.k)  # [1, Hkv, cap*64, 128]
    # the cache holds the appended tokens unchanged
    assert torch.equal(full["kc"][:, :, :nkb * 64].view(torch.int16), ch.k[:, :, :nkb * 64].view(torch.int16))
    assert torch.equal(full["vc"][:, :, :nkb * 64].view(torch.int16), ch.v[:, :, :nkb * 64].view(torch.int16))
    # block means of every cached block
    khat_ref = oracle.block_mean(np.ascontiguousarray(kbits[:, :, :nkb * 64].transpose(0, 2, 1, 3)))  # [1, Hkv, nkb, 128]
    assert float_bits_equal(f32(full["kmean"][:, :nkb]).reshape(1, HKV, nkb, 128), khat_ref)
    # pooled queries, scores, per-row masks, union and tables
    qhat_ref = oracle.block_mean(bits(ch.q))
    assert float_bits_equal(f32(full["qhat"]), qhat_ref)
    khat = np.zeros((1, HKV, cap, 128), dtype=np.float32)
    khat[:, :, :nkb] = khat_ref
    sc = oracle.block_scores(qhat_ref, khat, P, full["scale"])
    keep = oracle.select_rows(sc, P, oracle.Rule(topk=TOPK, sink_blocks=1, local_blocks=2))
    assert np.array_equal(unpack_rowmask(full["rowmask"], cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, HKV, P)
    assert np.array_equal(full["counts"].cpu().numpy(), ref_cnt)
    assert np.array_equal(full["table"].cpu().numpy(), ref_tab)


def test_fullsize_table_structure(full):
    P, cap = full["P"][0], full["cap"]
    qb = LQ // 64
    table = full["table"].cpu().numpy()
    counts = full["counts"].cpu().numpy()
    for r in range(HKV):
        n = int(counts[r])
        row = table[r, :n]
        assert qb < n <= P + qb
        assert (np.diff(row) > 0).all()  # strictly ascending, unique
        assert np.array_equal(row[-qb:], np.arange(P, P + qb))  # the chunk's blocks close the row
        assert row[0] == 0  # sink block
        assert {P - 2, P - 1} <= set(row.tolist())  # the 2 local blocks
        # every query row keeps at least top-k past blocks, so the union keeps at least k
        assert n - qb >= TOPK
    keep = (counts - qb).sum() / (HKV * P)
    assert 0.15 < keep < 0.40, keep  # the planted inputs give about a quarter at k = 10


def test_fullsize_attention_sampled_rows(full):
    ch, P, cap = full["ch"], full["P"], full["cap"]
    out, lse = ops.attn_fwd(ch.q, full["K"], full["V"], full["table"], full["counts"], P, full["scale"], cap, HKV,
                            with_lse=True)
    torch.cuda.synchronize()
    got, got_lse = f32(out), f32(lse)
    assert np.isfinite(got).all()
    qbits, kbits, vbits = bits(ch.q), bits(ch.k), bits(ch.v)
    table, counts = full["table"].cpu().numpy(), full["counts"].cpu().numpy()
    for q0, q1 in [(0, 8), (LQ - 8, LQ)]:
        ref, ref_lse = oracle.attention(qbits, kbits, vbits, P, table, counts, full["scale"], with_lse=True,
                                        q_range=(q0, q1))
        err = np.abs(got[:, q0:q1] - ref[:, q0:q1])
        assert err.max() <= ATOL_MAX, (q0, err.max())
        assert err.mean() <= ATOL_MEAN, (q0, err.mean())
        lerr = np.abs(got_lse[:, :, q0:q1] - ref_lse[:, :, q0:q1])
        assert lerr.max() <= 4e-3, (q0, lerr.max())


@pytest.mark.parametrize("forced", [1, 3])
def test_fullsize_split_plan_matches_unsplit(full, forced):
    """The automatic plan (one launch, 128-row tiles whose two key groups split each row's
    list inside the workgroup) against forced splits of the key range through HBM partials
    and the merge kernel."""
    ch, P, cap = full["ch"], full["P"], full["cap"]
    args = (ch.q, full["K"], full["V"], full["table"], full["counts"], P, full["scale"], cap, HKV)
    auto = ops.attn_fwd(*args, num_splits=0)
    other = ops.attn_fwd(*args, num_splits=forced)
    torch.cuda.synchronize()
    # the split plan changes only where the online softmax rescales and the merge's rounding:
    # a few bf16 ulps at most, on a small share of the outputs
    d = (other.float() - auto.float()).abs()
    assert d.max().item() <= ATOL_MAX and d.mean().item() <= 2e-4, (d.max().item(), d.mean().item())


def _check_sampled_attention(q, k, v, P, table, counts, cap, hkv, scale, samples):
    """Attention of the sampled query tokens against the oracle over the same tables."""
    out, lse = ops.attn_fwd(q, ops.KV.heads_first(k), ops.KV.heads_first(v), table, counts, P, scale, cap, hkv,
                            with_lse=True)
    torch.cuda.synchronize()
    got, got_lse = f32(out), f32(lse)
    assert np.isfinite(got).all()
    qbits, kbits, vbits = bits(q), bits(k), bits(v)
    tab, cnt = table.cpu().numpy(), counts.cpu().numpy()
    for q0, q1 in samples:
        ref, ref_lse = oracle.attention(qbits, kbits, vbits, P, tab, cnt, scale, with_lse=True, q_range=(q0, q1))
        err = np.abs(got[:, q0:q1] - ref[:, q0:q1])
        assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (q0, err.max(), err.mean())
        assert np.abs(got_lse[:, :, q0:q1] - ref_lse[:, :, q0:q1]).max() <= 4e-3


def test_fullsize_config1_attngate(gpu):
    """Config 1: 32768 cached tokens of which the last 1024 are the chunk (P = 496), 32 / 8
    heads, AttnGate (mean-pooled Q and K, per-head 128x128 projections ~ N(0, 0.02), block
    RoPE), softmax threshold 5e-3 + sink block + 2 local blocks."""
    from compactattention_amd.synthetic import rope_tables

    print("case: full-size config 1 (AttnGate, 32768 tokens, chunk 1024)", flush=True)
    past, lq, hq, hkv = 31744, 1024, 32, 8
    ch = make_chunk_device(past, lq, hq, hkv, gpu)
    cap, P = ch.kv_cap, ch.past_blocks
    g = torch.Generator().manual_seed(1234)
    wq = (torch.randn((hq, 128, 128), generator=g) * 0.02).float()
    wk = (torch.randn((hkv, 128, 128), generator=g) * 0.02).float()
    cos, sin = rope_tables(cap)
    kc, vc = torch.zeros_like(ch.k), torch.zeros_like(ch.v)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((hkv, cap, 128), dtype=torch.float32, device=gpu)
    kgate = torch.zeros_like(kmean)
    gate = dict(gate_wk=wk.to(gpu), rope_cos=cos.to(gpu), rope_sin=sin.to(gpu), kgate=kgate)
    for t0 in range(0, past, 16384):
        t1 = min(past, t0 + 16384)
        ops.cache_fill(ch.k[:, :, t0:t1].transpose(1, 2).contiguous(), ch.v[:, :, t0:t1].transpose(1, 2).contiguous(),
                       K, V, [t0 // 64], cap, kmean, **gate)
    ops.cache_fill(ch.k[:, :, past:past + lq].transpose(1, 2).contiguous(),
                   ch.v[:, :, past:past + lq].transpose(1, 2).contiguous(), K, V, P, cap, kmean, **gate)
    scale = 1.0 / math.sqrt(128)
    rule = ops.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2)
    qhat = ops.pool_query(ch.q, P, cap, gate_wq=wq.to(gpu), rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
    rowmask, _ = ops.score_select(qhat, kgate, scale, rule, P, hkv, cap)
    table, counts, _, _ = ops.union_compact(rowmask, P, hkv, cap)
    torch.cuda.synchronize()
    nkb = P[0] + lq // 64
    means = oracle.block_mean(np.ascontiguousarray(bits(ch.k)[:, :, :nkb * 64].transpose(0, 2, 1, 3)))
    khat = np.zeros((1, hkv, cap, 128), dtype=np.float32)
    khat[:, :, :nkb] = oracle.gate_project(means, f32(wk), f32(cos), f32(sin), [0])
    assert float_bits_equal(f32(kgate[:, :nkb]).reshape(1, hkv, nkb, 128), khat[:, :, :nkb])
    qref = oracle.gate_project(oracle.block_mean(bits(ch.q)), f32(wq), f32(cos), f32(sin), P)
    assert float_bits_equal(f32(qhat), qref)
    keep = oracle.select_rows(oracle.block_scores(qref, khat, P, scale), P,
                              oracle.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2))
    assert np.array_equal(unpack_rowmask(rowmask, cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, hkv, P)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)
    _check_sampled_attention(ch.q, kc, vc, P, table, counts, cap, hkv, scale, [(0, 8), (lq - 8, lq)])


def test_fullsize_config4_ragged(gpu):
    """Config 4: four requests with cached pasts 16384 / 49152 / 98304 / 131072 tokens, a
    512-token chunk each in one launch per kernel, 28 / 4 heads (G = 7), FlashPrefill pooled
    top-k 3 + sink block + 2 local blocks (about 20 % of the past blocks after the union)."""
    print("case: full-size config 4 (ragged batch, G = 7)", flush=True)
    pasts, lq, hq, hkv = (16384, 49152, 98304, 131072), 512, 28, 4
    B, qb = len(pasts), lq // 64
    P = [p // 64 for p in pasts]
    cap = max(P) + qb
    chs = [make_chunk_device(p, lq, hq, hkv, gpu, seed=1234 + i, kv_cap=cap) for i, p in enumerate(pasts)]
    q = torch.cat([c.q for c in chs], 0)
    k = torch.cat([c.k for c in chs], 0)  # [B, Hkv, cap*64, 128], zero past each request's end
    v = torch.cat([c.v for c in chs], 0)
    del chs
    kmean = torch.zeros((B * hkv, cap, 128), dtype=torch.float32, device=gpu)
    for b in range(B):
        ops.cache_fill(k[b:b + 1, :, :(P[b] + qb) * 64].transpose(1, 2).contiguous(), None, None, None, [0], cap,
                       kmean[b * hkv:(b + 1) * hkv])
    scale = 1.0 / math.sqrt(128)
    rule = ops.Rule(topk=3, sink_blocks=1, local_blocks=2)
    qhat = ops.pool_query(q, P, cap)
    rowmask, _ = ops.score_select(qhat, kmean, scale, rule, P, hkv, cap)
    table, counts, _, _ = ops.union_compact(rowmask, P, hkv, cap)
    torch.cuda.synchronize()
    kbits = bits(k)
    khat = np.zeros((B, hkv, cap, 128), dtype=np.float32)
    for b in range(B):
        n = P[b] + qb
        khat[b, :, :n] = oracle.block_mean(np.ascontiguousarray(kbits[b:b + 1, :, :n * 64].transpose(0, 2, 1, 3)))[0]
    assert float_bits_equal(f32(kmean).reshape(B, hkv, cap, 128), khat)
    qref = oracle.block_mean(bits(q))
    assert float_bits_equal(f32(qhat), qref)
    keep = oracle.select_rows(oracle.block_scores(qref, khat, P, scale), P,
                              oracle.Rule(topk=3, sink_blocks=1, local_blocks=2))
    assert np.array_equal(unpack_rowmask(rowmask, cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, hkv, P)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)
    kept = [float(((counts.cpu().view(B, hkv)[b] - qb).float() / P[b]).mean()) for b in range(B)]
    assert all(0.05 < r < 0.5 for r in kept), kept
    _check_sampled_attention(q, k, v, P, table, counts, cap, hkv, scale, [(0, 4), (lq - 4, lq)])
