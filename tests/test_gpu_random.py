"""Seeded random chunk steps through the whole path, against the CPU oracle.

Each case draws a batch (1-4 requests of different past lengths), a GQA shape (1-4 KV heads,
group 1-8), a chunk of 64-256 tokens, a KV layout (heads-first, seq-first or a permuted page
pool), a selection rule and a split count, then runs the library's chunk step:
  ca_cache_fill (ragged append + mean-K) -> ca_pool_query -> ca_score_select ->
  ca_union_compact -> ca_attn_fwd,
and checks the cache contents, block means, pooled queries, scores, per-row masks, tables
and counts bit for bit, and the attention output and log-sum-exp within the north-star
tolerance (max-abs 2e-2, mean-abs 2e-3) of the fp64 oracle over the same tables.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from compactattention_amd import ops
from compactattention_amd.synthetic import make_chunk

from .util import bits, f32, float_bits_equal, unpack_rowmask

pytestmark = pytest.mark.gpu

ATOL_MAX = 2e-2
ATOL_MEAN = 2e-3
SEEDS = list(range(40))


def _rule(rng) -> oracle.Rule:
    kind = int(rng.integers(0, 6))
    sink = int(rng.integers(0, 3))
    if kind == 0:
        return oracle.Rule(topk=int(rng.integers(1, 9)), sink_blocks=sink, local_blocks=int(rng.integers(0, 3)))
    if kind == 1:
        return oracle.Rule(alpha=float(rng.choice([0.06, 0.2, 0.5])), sink_blocks=sink,
                           window_blocks=int(rng.integers(0, 5)))
    if kind == 2:
        return oracle.Rule(threshold=float(rng.choice([1e-3, 5e-3, 2e-2])), sink_blocks=sink,
                           local_blocks=int(rng.integers(0, 3)))
    if kind == 3:
        return oracle.Rule(topk=int(rng.integers(1, 6)), alpha=float(rng.choice([0.3, 0.6])))
    if kind == 4:  # the reference's min_budget: top-k over all columns of the zeroed row
        return oracle.Rule(topk=int(rng.integers(1, 12)), alpha=0.06, sink_blocks=sink,
                           window_blocks=int(rng.integers(0, 5)), topk_all_columns=True)
    return oracle.Rule(topk=int(rng.integers(1, 6)), sink_blocks=1, local_blocks=2,
                       last_n_block=int(rng.integers(0, 3)))


def _ops_rule(r: oracle.Rule) -> ops.Rule:
    return ops.Rule(topk=r.topk, alpha=r.alpha, threshold=r.threshold, sink_blocks=r.sink_blocks,
                    window_blocks=r.window_blocks, local_blocks=r.local_blocks, last_n_block=r.last_n_block,
                    topk_all_columns=r.topk_all_columns)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_chunk_step(gpu, seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 5))
    Hkv = int(rng.choice([1, 2, 3, 4]))
    G = int(rng.choice([1, 2, 3, 4, 7, 8]))
    Hq = Hkv * G
    Lq = 64 * int(rng.integers(1, 5))
    qb = Lq // 64
    past = [int(x) for x in rng.integers(0, 48, size=B)]
    cap = max(past) + qb + int(rng.integers(0, 4))
    layout = str(rng.choice(["heads_first", "seq_first", "paged"]))
    splits = int(rng.choice([0, 0, 1, 2, 3]))
    rule = _rule(rng)
    print(f"case: random chunk step seed={seed} B={B} Hkv={Hkv} G={G} Lq={Lq} past={past} cap={cap} "
          f"layout={layout} splits={splits} rule={rule}", flush=True)

    ch = make_chunk([64 * p for p in past], Lq, Hq, Hkv, seed=2000 + seed, planted_blocks=2, kv_cap=cap)
    rows = B * Hkv
    # the cache holds each request's past; the chunk is appended by ca_cache_fill
    kpast = ch.k.clone()
    vpast = ch.v.clone()
    for b, P in enumerate(past):
        kpast[b, :, 64 * P:] = 0
        vpast[b, :, 64 * P:] = 0
    if layout == "heads_first":
        kc, vc = kpast.to(gpu), vpast.to(gpu)
        K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    elif layout == "seq_first":
        kc, vc = kpast.transpose(1, 2).contiguous().to(gpu), vpast.transpose(1, 2).contiguous().to(gpu)
        K, V = ops.KV.seq_first(kc), ops.KV.seq_first(vc)
    else:
        g = torch.Generator().manual_seed(seed)
        perm = torch.randperm(rows * cap, generator=g).to(torch.int32).view(rows, cap)
        pool_k = torch.zeros((rows * cap, 64, 128), dtype=torch.bfloat16)
        pool_v = torch.zeros_like(pool_k)
        pool_k[perm.view(-1).long()] = kpast.view(rows, cap, 64, 128).reshape(rows * cap, 64, 128)
        pool_v[perm.view(-1).long()] = vpast.view(rows, cap, 64, 128).reshape(rows * cap, 64, 128)
        kc, vc, pt = pool_k.to(gpu), pool_v.to(gpu), perm.to(gpu)
        K, V = ops.KV.paged(kc, pt), ops.KV.paged(vc, pt)

    # past block means from the past tokens (summaries only), then the chunk step
    kmean = torch.full((rows, cap, 128), float("nan"), dtype=torch.float32, device=gpu)
    for b, P in enumerate(past):
        if P > 0:
            kp = ch.k[b:b + 1, :, :64 * P].transpose(1, 2).contiguous().to(gpu)
            ops.cache_fill(kp, None, None, None, [0], cap, kmean[b * Hkv:(b + 1) * Hkv])
    k_new = torch.stack([ch.k[b, :, 64 * P:64 * P + Lq] for b, P in enumerate(past)]).transpose(1, 2).contiguous()
    v_new = torch.stack([ch.v[b, :, 64 * P:64 * P + Lq] for b, P in enumerate(past)]).transpose(1, 2).contiguous()
    ops.cache_fill(k_new.to(gpu), v_new.to(gpu), K, V, past, cap, kmean)
    qg = ch.q.to(gpu)
    qhat = ops.pool_query(qg, past, cap)
    scale = 1.0 / math.sqrt(128)
    rowmask, scores = ops.score_select(qhat, kmean, scale, _ops_rule(rule), past, Hkv, cap, with_scores=True)
    table, counts, _, _ = ops.union_compact(rowmask, past, Hkv, cap, last_n_block=rule.last_n_block)
    out, lse = ops.attn_fwd(qg, K, V, table, counts, past, scale, cap, Hkv, with_lse=True, num_splits=splits)
    torch.cuda.synchronize()

    # cache contents: every live token of every row where its layout puts it
    if layout == "heads_first":
        got_k, got_v = kc.cpu(), vc.cpu()
    elif layout == "seq_first":
        got_k, got_v = kc.cpu().transpose(1, 2), vc.cpu().transpose(1, 2)
    else:
        idx = perm.view(-1).long()
        got_k = kc.cpu()[idx].view(B, Hkv, cap * 64, 128)
        got_v = vc.cpu()[idx].view(B, Hkv, cap * 64, 128)
    for b, P in enumerate(past):
        live = 64 * (P + qb)
        assert torch.equal(got_k[b, :, :live], ch.k[b, :, :live])
        assert torch.equal(got_v[b, :, :live], ch.v[b, :, :live])

    kbits = bits(ch.k)
    khat = np.zeros((B, Hkv, cap, 128), dtype=np.float32)
    km = f32(kmean).reshape(B, Hkv, cap, 128)
    for b, P in enumerate(past):
        n = P + qb
        khat[b, :, :n] = oracle.block_mean(np.ascontiguousarray(kbits[b:b + 1, :, :n * 64].transpose(0, 2, 1, 3)))[0]
        assert float_bits_equal(km[b, :, :n], khat[b, :, :n])
    qref = oracle.block_mean(bits(ch.q))
    assert float_bits_equal(f32(qhat), qref)
    ref_scores = oracle.block_scores(qref, khat, past, scale)
    assert float_bits_equal(f32(scores), ref_scores)
    keep = oracle.select_rows(ref_scores, past, rule)
    assert np.array_equal(unpack_rowmask(rowmask, cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, Hkv, past, rule.last_n_block)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)

    ref, ref_lse = oracle.attention(bits(ch.q), kbits, bits(ch.v), past, ref_tab, ref_cnt, scale, with_lse=True)
    got = f32(out)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert err.max() <= ATOL_MAX, err.max()
    assert err.mean() <= ATOL_MEAN, err.mean()
    lerr = np.abs(f32(lse) - ref_lse)
    assert lerr.max() <= 4e-3, lerr.max()


@pytest.mark.parametrize("seed", list(range(24)))
def test_random_decode_step(gpu, seed):
    """Dense decode over whole caches of unaligned lengths: 1-4 requests, 1-8 query rows each
    (the last positions of kv_len), G up to 16, three KV layouts, automatic and forced split
    counts; slots past each kv_len hold NaN and must not reach the result."""
    rng = np.random.default_rng(5000 + seed)
    B = int(rng.integers(1, 5))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 7, 16]))
    Hq = Hkv * G
    Lq = int(rng.integers(1, 9))
    kv_len = [int(x) for x in rng.integers(Lq, 4000, size=B)]
    cap = (max(kv_len) + 63) // 64 + int(rng.integers(0, 3))
    layout = str(rng.choice(["heads_first", "seq_first", "paged"]))
    splits = int(rng.choice([0, 0, 1, 3, 7]))
    print(f"case: random decode seed={seed} B={B} Hkv={Hkv} G={G} Lq={Lq} kv_len={kv_len} cap={cap} "
          f"layout={layout} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(6000 + seed)
    q = torch.randn((B, Lq, Hq, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16)
    for b, n in enumerate(kv_len):
        k[b, :, n:] = float("nan")
        v[b, :, n:] = float("nan")
    if layout == "heads_first":
        K, V = ops.KV.heads_first(k.to(gpu)), ops.KV.heads_first(v.to(gpu))
    elif layout == "seq_first":
        K = ops.KV.seq_first(k.transpose(1, 2).contiguous().to(gpu))
        V = ops.KV.seq_first(v.transpose(1, 2).contiguous().to(gpu))
    else:
        rows = B * Hkv
        perm = torch.randperm(rows * cap, generator=g).to(torch.int32).view(rows, cap)
        pool_k = torch.full((rows * cap, 64, 128), float("nan"), dtype=torch.bfloat16)
        pool_v = torch.full_like(pool_k, float("nan"))
        pool_k[perm.view(-1).long()] = k.reshape(rows * cap, 64, 128)
        pool_v[perm.view(-1).long()] = v.reshape(rows * cap, 64, 128)
        K, V = ops.KV.paged(pool_k.to(gpu), perm.to(gpu)), ops.KV.paged(pool_v.to(gpu), perm.to(gpu))
    scale = 1.0 / math.sqrt(128)
    out, lse = ops.attn_decode(q.to(gpu), K, V, kv_len, scale, cap, Hkv, with_lse=True, num_splits=splits)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.attention_decode(bits(q), bits(k), bits(v), kv_len, scale, with_lse=True)
    got = f32(out)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert err.max() <= ATOL_MAX, err.max()
    assert err.mean() <= ATOL_MEAN, err.mean()
    lerr = np.abs(f32(lse) - ref_lse)
    assert lerr.max() <= 4e-3, lerr.max()
