"""GPU parity of every C-ABI entry point against the CPU oracle.

Bit-exact: cache copy, mean-K / gate-K summaries, pooled Q, fp32 block scores, per-row
selection masks, unions, block tables and counts.  Tolerance (north star): attention
output in bf16 within max-abs 2e-2 and mean-abs 2e-3 of the fp64-accumulated oracle over
the same selected blocks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from compactattention_amd import ops
from compactattention_amd.synthetic import make_chunk, rope_tables

from .util import bits, f32, float_bits_equal, pack_rowmask, torch_reference_check, unpack_rowmask

pytestmark = pytest.mark.gpu

ATOL_MAX = 2e-2
ATOL_MEAN = 2e-3


def _print_case(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# ----------------------------------------------------------------------------- cache fill
@pytest.mark.parametrize("layout", ["heads_first", "seq_first", "paged"])
@pytest.mark.parametrize("gate", [False, True])
def test_cache_fill_bit_exact(gpu, layout, gate):
    _print_case(test="cache_fill", layout=layout, gate=gate)
    B, Lq, Hkv, past = 2, 256, 3, [5, 9]
    qb = Lq // 64
    cap = max(past) + qb + 2
    g = torch.Generator().manual_seed(7)
    k_new = torch.randn((B, Lq, Hkv, 128), generator=g).to(torch.bfloat16)
    v_new = torch.randn((B, Lq, Hkv, 128), generator=g).to(torch.bfloat16)
    wk = (torch.randn((Hkv, 128, 128), generator=g) * 0.02).float()
    cos, sin = rope_tables(cap)
    if layout == "heads_first":
        kc = torch.zeros((B, Hkv, cap * 64, 128), dtype=torch.bfloat16, device=gpu)
        vc = torch.zeros_like(kc)
        K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    elif layout == "seq_first":
        kc = torch.zeros((B, cap * 64, Hkv, 128), dtype=torch.bfloat16, device=gpu)
        vc = torch.zeros_like(kc)
        K, V = ops.KV.seq_first(kc), ops.KV.seq_first(vc)
    else:
        rows = B * Hkv
        perm = torch.randperm(rows * cap, generator=g).to(torch.int32)
        pt = perm.view(rows, cap).contiguous().to(gpu)
        kc = torch.zeros((rows * cap, 64, 128), dtype=torch.bfloat16, device=gpu)
        vc = torch.zeros_like(kc)
        K, V = ops.KV.paged(kc, pt), ops.KV.paged(vc, pt)
    kmean = torch.full((B * Hkv, cap, 128), float("nan"), device=gpu)
    kgate = torch.full((B * Hkv, cap, 128), float("nan"), device=gpu) if gate else None
    ops.cache_fill(k_new.to(gpu), v_new.to(gpu), K, V, past, cap, kmean,
                   gate_wk=wk.to(gpu) if gate else None, rope_cos=cos.to(gpu) if gate else None,
                   rope_sin=sin.to(gpu) if gate else None, kgate=kgate)
    torch.cuda.synchronize()
    # copy: every new block lands at its logical position
    for b in range(B):
        for h in range(Hkv):
            for j in range(qb):
                kb = past[b] + j
                if layout == "heads_first":
                    got_k = kc[b, h, kb * 64:(kb + 1) * 64]
                    got_v = vc[b, h, kb * 64:(kb + 1) * 64]
                elif layout == "seq_first":
                    got_k = kc[b, kb * 64:(kb + 1) * 64, h]
                    got_v = vc[b, kb * 64:(kb + 1) * 64, h]
                else:
                    page = int(pt[b * Hkv + h, kb])
                    got_k, got_v = kc[page], vc[page]
                assert torch.equal(got_k.cpu(), k_new[b, j * 64:(j + 1) * 64, h])
                assert torch.equal(got_v.cpu(), v_new[b, j * 64:(j + 1) * 64, h])
    means = oracle.block_mean(bits(k_new))  # [B, Hkv, qb, 128]
    km = f32(kmean).reshape(B, Hkv, cap, 128)
    for b in range(B):
        assert float_bits_equal(km[b, :, past[b]:past[b] + qb], means[b])
    if gate:
        kg = f32(kgate).reshape(B, Hkv, cap, 128)
        ref = oracle.gate_project(means, f32(wk), f32(cos), f32(sin), past)
        for b in range(B):
            assert float_bits_equal(kg[b, :, past[b]:past[b] + qb], ref[b])


@pytest.mark.parametrize("Lq", [37, 128 + 29])
@pytest.mark.parametrize("layout", ["heads_first", "paged"])
def test_partial_last_block(gpu, layout, Lq):
    """A chunk whose length is not a multiple of 64 (ceil(Lq/64) blocks, the last holding
    Lq % 64 tokens): the cache receives exactly its Lq rows (the rows past them keep their NaN
    fill), the mean-K / query means / AttnGate pools of the partial block cover its valid
    tokens (bit-exact against the oracle's restatement of compute_mean_vector and the ceil_mode
    pools), and attention over tables that end in the partial block never reads past the
    chunk (its NaN rows would poison the output) -- against the fp64 oracle."""
    _print_case(test="partial_last_block", layout=layout, Lq=Lq)
    B, Hkv, G, past = 2, 2, 3, [3, 7]
    Hq = Hkv * G
    qb = -(-Lq // 64)
    cap = max(past) + qb
    g = torch.Generator().manual_seed(Lq)
    k_new = torch.randn((B, Lq, Hkv, 128), generator=g).to(torch.bfloat16)
    v_new = torch.randn((B, Lq, Hkv, 128), generator=g).to(torch.bfloat16)
    q = torch.randn((B, Lq, Hq, 128), generator=g).to(torch.bfloat16)
    k_past = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16)
    v_past = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16)
    nan = float("nan")
    if layout == "heads_first":
        kc = torch.full((B, Hkv, cap * 64, 128), nan, dtype=torch.bfloat16)
        vc = kc.clone()
        for b in range(B):  # the past as it sits in the cache
            kc[b, :, :64 * past[b]] = k_past[b, :, :64 * past[b]]
            vc[b, :, :64 * past[b]] = v_past[b, :, :64 * past[b]]
        kc, vc = kc.to(gpu), vc.to(gpu)
        K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    else:
        rows = B * Hkv
        pt = torch.randperm(rows * cap, generator=g).to(torch.int32).view(rows, cap).contiguous()
        kc = torch.full((rows * cap, 64, 128), nan, dtype=torch.bfloat16)
        vc = kc.clone()
        for b in range(B):
            for h in range(Hkv):
                for kb in range(past[b]):
                    kc[int(pt[b * Hkv + h, kb])] = k_past[b, h, 64 * kb:64 * kb + 64]
                    vc[int(pt[b * Hkv + h, kb])] = v_past[b, h, 64 * kb:64 * kb + 64]
        kc, vc, pt = kc.to(gpu), vc.to(gpu), pt.to(gpu)
        K, V = ops.KV.paged(kc, pt), ops.KV.paged(vc, pt)
    kmean = torch.full((B * Hkv, cap, 128), nan, device=gpu)
    qhat = ops.cache_fill_pool_query(k_new.to(gpu), v_new.to(gpu), K, V, past, cap, kmean, q.to(gpu))
    torch.cuda.synchronize()
    # cache rows: the chunk's Lq rows at 64 * past[b], NaN after them
    for b in range(B):
        for h in range(Hkv):
            if layout == "heads_first":
                got_k = kc[b, h, 64 * past[b]:64 * (past[b] + qb)].cpu()
            else:
                got_k = torch.cat([kc[int(pt[b * Hkv + h, past[b] + j])].cpu() for j in range(qb)])
            assert torch.equal(got_k[:Lq], k_new[b, :, h])
            assert torch.isnan(got_k[Lq:].float()).all()
    km = f32(kmean).reshape(B, Hkv, cap, 128)
    means = oracle.block_mean(bits(k_new))
    assert means.shape[2] == qb
    for b in range(B):
        assert float_bits_equal(km[b, :, past[b]:past[b] + qb], means[b])
    assert float_bits_equal(f32(qhat), oracle.block_mean(bits(q)))
    # AttnGate pools of the partial blocks (max, min, avg), projected per KV head and rotated
    pools = ops.POOL_BITS["max"] | ops.POOL_BITS["min"] | ops.POOL_BITS["avg"]
    wk = (torch.randn((Hkv, 3 * 128, 128), generator=g) * 0.02).float()
    wq = (torch.randn((Hq, 128, 128), generator=g) * 0.02).float()
    cos, sin = rope_tables(cap)
    kgate = torch.full((B, Hkv, cap, 128), nan, device=gpu)
    ops.gate_key_summaries(k_new.to(gpu), past, cap, pools, wk.to(gpu), kgate, rope_cos=cos.to(gpu),
                           rope_sin=sin.to(gpu))
    gq = ops.gate_query_summaries(q.to(gpu), past, cap, ops.POOL_BITS["avg"], wq.to(gpu), Hkv, rope_cos=cos.to(gpu),
                                  rope_sin=sin.to(gpu))
    ref_k = oracle.gate_project(oracle.block_pool(bits(k_new), pools), f32(wk), f32(cos), f32(sin), past)
    ref_q = oracle.gate_project(oracle.block_mean(bits(q)), f32(wq), f32(cos), f32(sin), past)
    kg = f32(kgate)
    for b in range(B):
        assert float_bits_equal(kg[b, :, past[b]:past[b] + qb], ref_k[b])
    assert float_bits_equal(f32(gq), ref_q)
    # attention over tables that end with the chunk's blocks (the partial one last)
    kv_tab = torch.zeros((B, Hkv, cap), dtype=torch.uint8)
    for b in range(B):
        kv_tab[b, :, :past[b]] = (torch.rand((Hkv, past[b]), generator=g) < 0.5).to(torch.uint8)
    table, counts = ops.compact_keep_kv(kv_tab.to(gpu), past, Lq, Hq, cap)
    out, lse = ops.attn_fwd(q.to(gpu), K, V, table, counts, past, 128 ** -0.5, cap, Hkv, with_lse=True)
    ktot = k_past.clone()
    vtot = v_past.clone()
    for b in range(B):
        ktot[b, :, 64 * past[b]:64 * past[b] + Lq] = k_new[b].transpose(0, 1)
        vtot[b, :, 64 * past[b]:64 * past[b] + Lq] = v_new[b].transpose(0, 1)
    ref, ref_lse = oracle.attention(bits(q), bits(ktot), bits(vtot), past, table.cpu().numpy(), counts.cpu().numpy(),
                                    128 ** -0.5, with_lse=True)
    got = f32(out)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())
    assert np.abs(f32(lse) - ref_lse).max() <= 4e-3


@pytest.mark.parametrize("layout", ["heads_first", "paged"])
def test_cache_fill_pool_query_equals_separate_calls(gpu, layout):
    """The one-launch chunk summaries (cache append + mean-K + query-block means) against
    ca_cache_fill and ca_pool_query called separately: cache, mean-K and qhat bit for bit,
    with the means also against the oracle; a ragged batch at G = 3."""
    _print_case(test="cache_fill_pool_query", layout=layout)
    B, Lq, Hkv, G, past = 2, 192, 2, 3, [4, 11]
    Hq = Hkv * G
    qb = Lq // 64
    cap = max(past) + qb + 1
    g = torch.Generator().manual_seed(23)
    k_new = torch.randn((B, Lq, Hkv, 128), generator=g).to(torch.bfloat16).to(gpu)
    v_new = torch.randn((B, Lq, Hkv, 128), generator=g).to(torch.bfloat16).to(gpu)
    q = torch.randn((B, Lq, Hq, 128), generator=g).to(torch.bfloat16).to(gpu)
    out = []
    for fused in (False, True):
        if layout == "heads_first":
            kc = torch.zeros((B, Hkv, cap * 64, 128), dtype=torch.bfloat16, device=gpu)
            vc = torch.zeros_like(kc)
            K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
        else:
            rows = B * Hkv
            pt = torch.randperm(rows * cap, generator=torch.Generator().manual_seed(5)).to(torch.int32)
            pt = pt.view(rows, cap).contiguous().to(gpu)
            kc = torch.zeros((rows * cap, 64, 128), dtype=torch.bfloat16, device=gpu)
            vc = torch.zeros_like(kc)
            K, V = ops.KV.paged(kc, pt), ops.KV.paged(vc, pt)
        kmean = torch.full((B * Hkv, cap, 128), float("nan"), device=gpu)
        if fused:
            qhat = ops.cache_fill_pool_query(k_new, v_new, K, V, past, cap, kmean, q)
        else:
            ops.cache_fill(k_new, v_new, K, V, past, cap, kmean)
            qhat = ops.pool_query(q, past, cap)
        torch.cuda.synchronize()
        out.append((kc.cpu(), vc.cpu(), f32(kmean), f32(qhat)))
    for a, b in zip(out[0], out[1]):
        if a.dtype == np.float32:
            assert float_bits_equal(a, b)
        else:
            assert torch.equal(a, b)
    assert float_bits_equal(out[1][3], oracle.block_mean(bits(q.cpu())))


# ----------------------------------------------------------------------------- pooled Q
@pytest.mark.parametrize("gate", [False, True])
def test_pool_query_bit_exact(gpu, gate):
    _print_case(test="pool_query", gate=gate)
    B, Lq, Hq, past = 2, 192, 5, [0, 7]
    g = torch.Generator().manual_seed(11)
    q = torch.randn((B, Lq, Hq, 128), generator=g).to(torch.bfloat16)
    wq = (torch.randn((Hq, 128, 128), generator=g) * 0.02).float()
    cap = max(past) + Lq // 64
    cos, sin = rope_tables(cap)
    qhat = ops.pool_query(q.to(gpu), past, cap, gate_wq=wq.to(gpu) if gate else None,
                          rope_cos=cos.to(gpu) if gate else None, rope_sin=sin.to(gpu) if gate else None)
    ref = oracle.block_mean(bits(q))
    if gate:
        ref = oracle.gate_project(ref, f32(wq), f32(cos), f32(sin), past)
    assert float_bits_equal(f32(qhat), ref)


# ----------------------------------------------------------------------------- AttnGate summaries
GATE_POOLS = [("avg",), ("max",), ("min", "avg"), ("max", "min", "avg")]


@pytest.mark.parametrize("per_q_head", [False, True])
@pytest.mark.parametrize("pools", GATE_POOLS, ids=lambda p: "".join(p))
def test_gate_key_summaries_bit_exact(gpu, pools, per_q_head):
    """K pools -> projection (per KV head, or per Q head on the K block repeated to the
    group's Q heads) -> block RoPE, bit for bit against the oracle."""
    _print_case(test="gate_key_summaries", pools=pools, per_q_head=per_q_head)
    B, Lq, Hkv, G, past = 2, 192, 2, 3, [4, 7]
    Hq = Hkv * G
    qb = Lq // 64
    cap = max(past) + qb + 1
    C = len(pools)
    gh = Hq if per_q_head else Hkv
    g = torch.Generator().manual_seed(31 + C)
    k_new = torch.randn((B, Lq, Hkv, 128), generator=g).to(torch.bfloat16)
    wk = (torch.randn((gh, C * 128, 128), generator=g) * 0.02).float()
    cos, sin = rope_tables(cap)
    kgate = torch.full((B, gh, cap, 128), float("nan"), device=gpu)
    ops.gate_key_summaries(k_new.to(gpu), past, cap, ops.pool_bits(pools), wk.to(gpu), kgate, num_q_heads=Hq,
                           rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
    pooled = oracle.block_pool(bits(k_new), oracle.pool_bits(pools))  # [B, Hkv, qb, C*128]
    if per_q_head:
        pooled = np.repeat(pooled, G, axis=1)
    ref = oracle.gate_project(pooled, f32(wk), f32(cos), f32(sin), past)
    got = f32(kgate)
    for b in range(B):
        assert float_bits_equal(got[b, :, past[b]:past[b] + qb], ref[b])
        assert np.isnan(got[b, :, :past[b]]).all()  # nothing outside the new blocks is written


@pytest.mark.parametrize("mode", ["none", "per_q_head", "kv_group_aware"])
@pytest.mark.parametrize("pools", GATE_POOLS, ids=lambda p: "".join(p))
def test_gate_query_summaries_bit_exact(gpu, pools, mode):
    """Q pools -> no projection / per-Q-head projection / kv-group-aware projection of the
    group's concatenated pooled heads -> block RoPE, bit for bit against the oracle."""
    if mode == "none" and len(pools) > 1:
        pytest.skip("several query pools always have a projection (attn_gate.py:80-86)")
    _print_case(test="gate_query_summaries", pools=pools, mode=mode)
    B, Lq, Hkv, G, past = 2, 128, 2, 4, [3, 10]
    Hq = Hkv * G
    qb = Lq // 64
    cap = max(past) + qb
    C = len(pools)
    g = torch.Generator().manual_seed(57 + C)
    q = torch.randn((B, Lq, Hq, 128), generator=g).to(torch.bfloat16)
    cos, sin = rope_tables(cap)
    pooled = oracle.block_pool(bits(q), oracle.pool_bits(pools))  # [B, Hq, qb, C*128]
    if mode == "none":
        got = ops.gate_query_summaries(q.to(gpu), past, cap, ops.pool_bits(pools), None, Hkv)
        assert float_bits_equal(f32(got), pooled)
        # no projection but the block RoPE (the reference's default gate): the identity
        # projection in the oracle reproduces the pooled vector exactly before the rotation
        got = ops.gate_query_summaries(q.to(gpu), past, cap, ops.pool_bits(pools), None, Hkv,
                                       rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
        eye = np.tile(np.eye(128, dtype=np.float32), (Hq, 1, 1))
        ref = oracle.gate_project(pooled, eye, f32(cos), f32(sin), past)
    elif mode == "per_q_head":
        wq = (torch.randn((Hq, C * 128, 128), generator=g) * 0.02).float()
        got = ops.gate_query_summaries(q.to(gpu), past, cap, ops.pool_bits(pools), wq.to(gpu), Hkv,
                                       rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
        ref = oracle.gate_project(pooled, f32(wq), f32(cos), f32(sin), past)
    else:
        wq = (torch.randn((Hkv, G * C * 128, 128), generator=g) * 0.02).float()
        got = ops.gate_query_summaries(q.to(gpu), past, cap, ops.pool_bits(pools), wq.to(gpu), Hkv,
                                       rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
        cat = pooled.reshape(B, Hkv, G, qb, C * 128).transpose(0, 1, 3, 2, 4).reshape(B, Hkv, qb, G * C * 128)
        ref = oracle.gate_project(cat, f32(wq), f32(cos), f32(sin), past)
    assert float_bits_equal(f32(got), ref)


# ----------------------------------------------------------------------------- scoring + selection
RULES = {
    "topk_sink_local": oracle.Rule(topk=5, sink_blocks=1, local_blocks=2),
    "alpha_sink_window": oracle.Rule(alpha=0.06, sink_blocks=2, window_blocks=4),
    "threshold": oracle.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2),
    "topk_alpha": oracle.Rule(topk=3, alpha=0.5),
    "topk_ge_candidates": oracle.Rule(topk=1000),
    # the reference's min_budget: top-k over all Kb columns of the zeroed row
    "allcols_alpha_sink_window": oracle.Rule(topk=5, alpha=0.06, sink_blocks=2, window_blocks=4,
                                             topk_all_columns=True),
    "allcols_near_kb": oracle.Rule(topk=40, topk_all_columns=True),
    "allcols_ge_kb": oracle.Rule(topk=1000, topk_all_columns=True),
}


def _ops_rule(r: oracle.Rule) -> ops.Rule:
    return ops.Rule(topk=r.topk, alpha=r.alpha, threshold=r.threshold, sink_blocks=r.sink_blocks,
                    window_blocks=r.window_blocks, local_blocks=r.local_blocks, last_n_block=r.last_n_block,
                    topk_all_columns=r.topk_all_columns)


@pytest.mark.parametrize("rule_name", sorted(RULES))
@pytest.mark.parametrize("G", [1, 4, 7])
def test_score_select_bit_exact(gpu, rule_name, G):
    rule = RULES[rule_name]
    _print_case(test="score_select", rule=rule_name, G=G)
    B, Hkv, Lq = 2, 2, 256
    Hq = Hkv * G
    past = [37, 70]
    cap = max(past) + Lq // 64 + 3
    g = torch.Generator().manual_seed(100 + G)
    qhat = torch.randn((B, Hq, Lq // 64, 128), generator=g) * 0.3
    khat = torch.randn((B * Hkv, cap, 128), generator=g) * 0.3
    scale = 1.0 / math.sqrt(128)
    rowmask, scores = ops.score_select(qhat.to(gpu), khat.to(gpu), scale, _ops_rule(rule), past, Hkv, cap,
                                       with_scores=True)
    ref_scores = oracle.block_scores(qhat.numpy(), khat.numpy().reshape(B, Hkv, cap, 128), past, scale)
    assert float_bits_equal(f32(scores), ref_scores)
    ref_keep = oracle.select_rows(ref_scores, past, rule)
    assert np.array_equal(unpack_rowmask(rowmask, cap), ref_keep)


@pytest.mark.parametrize("past", [250, 1050, 2050, 3050, 4990])
def test_score_select_row_lengths(gpu, past):
    """Rows in every dispatch bucket of the selection kernel (the row held in 4, 8, 12 or 16
    registers per thread, and the LDS-staged kernel beyond 4096 blocks): scores and masks bit
    for bit, for the past-only and the all-columns top-k."""
    _print_case(test="score_select_rows", past=past)
    B, Hkv, G, Lq = 1, 1, 2, 128
    Hq = Hkv * G
    cap = past + Lq // 64 + 1
    scale = 1.0 / math.sqrt(128)
    g = torch.Generator().manual_seed(past)
    qhat = torch.randn((B, Hq, Lq // 64, 128), generator=g)
    khat = torch.randn((B * Hkv, cap, 128), generator=g)
    ref_scores = oracle.block_scores(qhat.numpy(), khat.numpy().reshape(B, Hkv, cap, 128), [past], scale)
    for rule in (oracle.Rule(topk=10, sink_blocks=1, local_blocks=2),
                 oracle.Rule(topk=24, alpha=0.5, window_blocks=3, topk_all_columns=True)):
        rowmask, scores = ops.score_select(qhat.to(gpu), khat.to(gpu), scale, _ops_rule(rule), [past], Hkv, cap,
                                           with_scores=True)
        assert float_bits_equal(f32(scores), ref_scores)
        assert np.array_equal(unpack_rowmask(rowmask, cap), oracle.select_rows(ref_scores, [past], rule))


@pytest.mark.parametrize("past,Hkv,G,Lq", [
    ([2048, 900], 4, 2, 1024),   # 8 rows x 2064 keys: 64 tiles per row, 16 of them of 33 keys
    ([4100, 3000], 2, 4, 256),   # 4 rows x 4104 keys: 128 tiles per row, 8 of 33 keys
])
def test_score_select_tiles_of_33_keys(gpu, past, Hkv, G, Lq):
    """Block logits whose 32-key tiles would overflow two workgroups per CU fit each row into
    fewer tiles, the first ones holding 33 keys; a shorter request's tiles end early.  Scores
    and masks bit for bit against the oracle."""
    _print_case(test="score_select_33", past=past, Hkv=Hkv, G=G)
    B = len(past)
    Hq = Hkv * G
    cap = max(past) + Lq // 64
    g = torch.Generator().manual_seed(sum(past))
    qhat = torch.randn((B, Hq, Lq // 64, 128), generator=g) * 0.3
    khat = torch.randn((B * Hkv, cap, 128), generator=g) * 0.3
    scale = 1.0 / math.sqrt(128)
    rule = oracle.Rule(topk=10, sink_blocks=1, local_blocks=2)
    rowmask, scores = ops.score_select(qhat.to(gpu), khat.to(gpu), scale, _ops_rule(rule), past, Hkv, cap,
                                       with_scores=True)
    ref_scores = oracle.block_scores(qhat.numpy(), khat.numpy().reshape(B, Hkv, cap, 128), past, scale)
    assert float_bits_equal(f32(scores), ref_scores)
    assert np.array_equal(unpack_rowmask(rowmask, cap), oracle.select_rows(ref_scores, past, rule))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_select_scores_ties_and_nonfinite(gpu, dtype):
    _print_case(test="select_scores", dtype=dtype)
    B, Hkv, G, Lq = 1, 2, 3, 128
    Hq = Hkv * G
    past = [50]
    qb = Lq // 64
    cap = 64
    g = torch.Generator().manual_seed(3)
    # few distinct values -> many ties; sprinkle -inf / nan / +inf / -0.0
    s = torch.randint(0, 4, (B, Hq, qb, cap), generator=g).float() * 0.25
    s[..., 3] = float("-inf")
    s[0, 1, 0, 7] = float("nan")
    s[0, 2, 1, 9] = float("inf")
    s[0, 0, 0, 11] = -0.0
    s = s.to(dtype)
    for rule in (oracle.Rule(topk=6), oracle.Rule(topk=6, alpha=0.9), oracle.Rule(threshold=0.3, sink_blocks=1),
                 oracle.Rule(topk=6, alpha=0.5, topk_all_columns=True), oracle.Rule(topk=51, topk_all_columns=True)):
        rowmask = ops.select_scores(s.to(gpu), _ops_rule(rule), past, Hkv, cap, Lq)
        ref = oracle.select_rows(s.float().numpy(), past, rule)
        assert np.array_equal(unpack_rowmask(rowmask, cap), ref), rule


@pytest.mark.parametrize("all_columns", [False, True])
@pytest.mark.parametrize("case", ["two_values", "k_gt_64", "k_eq_64", "sparse_finite", "negative"])
def test_select_topk_search_paths(gpu, case, all_columns):
    """Top-k through each branch of the kernel's search: the candidate list after the
    lane-maximum bound (k <= 64), its overflow into the full-row search (heavy ties) and
    k > 64; also rows where few lanes hold finite candidates and all-negative scores (where
    the all-columns form ranks the zeroed non-causal columns above every causal one)."""
    _print_case(test="select_topk_paths", case=case, all_columns=all_columns)
    B, Hkv, G, Lq = 1, 2, 2, 128
    Hq = Hkv * G
    past = [700]
    qb = Lq // 64
    cap = past[0] + qb
    g = torch.Generator().manual_seed(17)
    k = 10
    if case == "two_values":  # ~350 keys equal to the maximum: the list overflows
        s = (torch.rand((B, Hq, qb, cap), generator=g) < 0.5).float()
    elif case == "k_gt_64":
        s = torch.rand((B, Hq, qb, cap), generator=g)
        k = 100
    elif case == "k_eq_64":
        s = torch.randint(0, 50, (B, Hq, qb, cap), generator=g).float()
        k = 64
    elif case == "sparse_finite":  # finite candidates only in lanes 0..9 of each 64
        s = torch.rand((B, Hq, qb, cap), generator=g)
        s[..., (torch.arange(cap) % 64) >= 10] = float("nan")
        k = 30
    else:
        s = -torch.rand((B, Hq, qb, cap), generator=g) * 5
        s[..., 5] = -0.0
        s[..., 6] = 0.0
    rule = oracle.Rule(topk=k, topk_all_columns=all_columns)
    rowmask = ops.select_scores(s.to(gpu), _ops_rule(rule), past, Hkv, cap, Lq)
    ref = oracle.select_rows(s.numpy(), past, rule)
    if not all_columns:
        assert ref[..., :past[0]].sum(axis=-1).max() == k
    assert np.array_equal(unpack_rowmask(rowmask, cap), ref)


# ----------------------------------------------------------------------------- union + tables
@pytest.mark.parametrize("last_n_block", [0, 2])
@pytest.mark.parametrize("G", [1, 4, 7])
def test_union_compact_bit_exact(gpu, G, last_n_block):
    _print_case(test="union_compact", G=G, last_n_block=last_n_block)
    B, Hkv, Lq = 3, 2, 256
    Hq = Hkv * G
    past = [0, 33, 95]
    qb = Lq // 64
    cap = max(past) + qb + 5
    g = torch.Generator().manual_seed(G)
    rowkeep = (torch.rand((B, Hq, qb, cap), generator=g) < 0.05).to(torch.uint8).numpy()
    for b in range(B):  # the selection never marks non-causal entries
        for q in range(qb):
            rowkeep[b, :, q, past[b] + q + 1:] = 0
    rm = pack_rowmask(rowkeep, cap)
    rowmask = torch.from_numpy(rm.view(np.int32)).to(gpu)
    table, counts, keep_block, keep_kv = ops.union_compact(rowmask, past, Hkv, cap, last_n_block=last_n_block,
                                                            want_keep_block=True, want_keep_kv=True)
    ref_kb, ref_kv, ref_tab, ref_cnt = oracle.union_compact(rowkeep, Hkv, past, last_n_block)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)
    assert np.array_equal(keep_block.cpu().numpy(), ref_kb)
    assert np.array_equal(keep_kv.cpu().numpy(), ref_kv)
    # the caller-mask entry point reproduces the same table from keep_kv
    t2, c2 = ops.compact_keep_kv(torch.from_numpy(ref_kv).to(gpu), past, Lq, Hq, cap)
    assert np.array_equal(c2.cpu().numpy(), ref_cnt)
    assert np.array_equal(t2.cpu().numpy(), ref_tab)


def test_dense_table(gpu):
    past = [0, 3, 17]
    t, c = ops.dense_table(past, 128, 8, 2, 24, gpu)
    t, c = t.cpu().numpy(), c.cpu().numpy()
    for b, P in enumerate(past):
        for h in range(2):
            r = b * 2 + h
            assert c[r] == P + 2
            assert np.array_equal(t[r, :P + 2], np.arange(P + 2))
            assert (t[r, P + 2:] == -1).all()


@pytest.mark.parametrize("B,Hkv,cap", [(3, 2, 40), (1, 8, 2064), (2, 3, 7)])
def test_table_to_csr_matches_reference_spec(gpu, B, Hkv, cap):
    """CSR page lists from the block tables equal the reference's torch spec applied to the
    keep mask itself (flashinfer_zero_copy_prefill.py:482-510): pages_per_row = keep.sum,
    kv_indptr = [0, cumsum], kv_indices = global_ids[keep] with global id row*cap + block."""
    _print_case(test="table_to_csr", B=B, Hkv=Hkv, cap=cap)
    g = torch.Generator().manual_seed(B * 100 + cap)
    qb = 1
    past = [int(x) for x in torch.randint(0, cap - qb + 1, (B,), generator=g)]
    keep_kv = (torch.rand((B, Hkv, cap), generator=g) < 0.3).to(torch.uint8)
    table, counts = ops.compact_keep_kv(keep_kv.to(gpu), past, 64 * qb, Hkv, cap)
    indptr, indices, last = ops.table_to_csr(table, counts, B, Hkv, cap, with_last_page_len=True)
    torch.cuda.synchronize()
    keep = keep_kv.numpy().astype(bool).copy()
    for b, P in enumerate(past):  # visible blocks: the past's selection + the chunk's blocks
        keep[b, :, P + qb:] = False
        keep[b, :, P:P + qb] = True
    keep_flat = keep.reshape(B * Hkv, cap)
    ref_ptr = np.concatenate([[0], np.cumsum(keep_flat.sum(axis=1))]).astype(np.int32)
    global_ids = np.arange(B * Hkv * cap, dtype=np.int32).reshape(B * Hkv, cap)
    ref_idx = global_ids[keep_flat]
    got_ptr = indptr.cpu().numpy()
    assert np.array_equal(got_ptr, ref_ptr)
    assert np.array_equal(indices.cpu().numpy()[:ref_ptr[-1]], ref_idx)
    assert (last.cpu().numpy() == 64).all()


# ----------------------------------------------------------------------------- attention
def _attn_case(gpu, past_tokens, Lq, Hq, Hkv, layout, splits, keep_frac, seed):
    ch = make_chunk(past_tokens, Lq, Hq, Hkv, seed=seed, planted_blocks=2)
    B = len(past_tokens)
    cap = ch.kv_cap
    g = torch.Generator().manual_seed(seed + 1)
    keep_kv = (torch.rand((B, Hkv, cap), generator=g) < keep_frac).to(torch.uint8)
    qg, kg, vg = ch.q.to(gpu), ch.k.to(gpu), ch.v.to(gpu)
    table, counts = ops.compact_keep_kv(keep_kv.to(gpu), ch.past_blocks, Lq, Hq, cap)
    if layout == "heads_first":
        K, V = ops.KV.heads_first(kg), ops.KV.heads_first(vg)
    elif layout == "seq_first":
        K, V = ops.KV.seq_first(kg.transpose(1, 2).contiguous()), ops.KV.seq_first(vg.transpose(1, 2).contiguous())
    else:
        rows = B * Hkv
        perm = torch.randperm(rows * cap, generator=g).to(torch.int32).view(rows, cap)
        pool_k = torch.empty((rows * cap, 64, 128), dtype=torch.bfloat16)
        pool_v = torch.empty_like(pool_k)
        kc, vc = ch.k.view(rows, cap, 64, 128), ch.v.view(rows, cap, 64, 128)
        pool_k[perm.view(-1).long()] = kc.reshape(rows * cap, 64, 128)
        pool_v[perm.view(-1).long()] = vc.reshape(rows * cap, 64, 128)
        K, V = ops.KV.paged(pool_k.to(gpu), perm.to(gpu)), ops.KV.paged(pool_v.to(gpu), perm.to(gpu))
    scale = 1.0 / math.sqrt(128)
    out, lse = ops.attn_fwd(qg, K, V, table, counts, ch.past_blocks, scale, cap, Hkv, with_lse=True,
                            num_splits=splits)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.attention(bits(ch.q), bits(ch.k), bits(ch.v), ch.past_blocks, table.cpu().numpy(),
                                    counts.cpu().numpy(), scale, with_lse=True)
    got = f32(out)
    err = np.abs(got - ref)
    assert np.isfinite(got).all()
    assert err.max() <= ATOL_MAX, err.max()
    assert err.mean() <= ATOL_MEAN, err.mean()
    # the kernel's row sums add the bf16-rounded probabilities the PV product uses, so its
    # log-sum-exp carries the bf16 rounding of P (relative 2^-9 per term, averaging out)
    lerr = np.abs(f32(lse) - ref_lse)
    assert lerr.max() <= 4e-3, lerr.max()


@pytest.mark.parametrize("splits", [1, 2, 3])
@pytest.mark.parametrize("layout", ["heads_first", "seq_first", "paged"])
def test_attention_layouts_and_splits(gpu, layout, splits):
    _print_case(test="attention", layout=layout, splits=splits)
    _attn_case(gpu, [64 * 40], 256, 8, 2, layout, splits, 0.3, seed=21)


@pytest.mark.parametrize("G,Lq", [(1, 128), (4, 320), (7, 256), (8, 192)])
def test_attention_groups(gpu, G, Lq):
    _print_case(test="attention_groups", G=G, Lq=Lq)
    _attn_case(gpu, [64 * 23], Lq, 2 * G, 2, "heads_first", 0, 0.4, seed=31 + G)


def test_attention_ragged_batch(gpu):
    _print_case(test="attention_ragged")
    _attn_case(gpu, [0, 64 * 5, 64 * 31, 64 * 12], 128, 14, 2, "heads_first", 0, 0.25, seed=41)


def test_attention_ragged_split_plan(gpu):
    """The automatic split count (here 12 for every request, the shortest request's lists
    being split down to a few blocks) through the LSE merge."""
    _print_case(test="attention_ragged_plan")
    _attn_case(gpu, [64 * 16, 64 * 60, 64 * 120, 64 * 200], 128, 8, 2, "heads_first", 0, 0.3, seed=43)


@pytest.mark.parametrize("layout", ["seq_first", "paged"])
def test_attention_ragged_rows_not_dividing_xcds(gpu, layout):
    """Nine KV rows (3 requests x 3 KV heads) of ragged lengths under the automatic plan:
    single splits dealt over the 8 XCDs, against the fp64 oracle in two more layouts."""
    _print_case(test="attention_ragged_9_rows", layout=layout)
    _attn_case(gpu, [64 * 10, 64 * 57, 64 * 120], 128, 6, 3, layout, 0, 0.35, seed=45)


@pytest.mark.parametrize("even", [True, False])
def test_attention_ragged_unsplit_choice(gpu, even):
    """A ragged launch with enough row tiles (4 requests x 2 KV rows x 24 tiles of 256 query
    rows) that the kernel picks between its split plan and one unsplit round from the
    selected counts: every row selecting the same number of blocks runs unsplit; dense
    tables over pasts of 16..128 blocks (largest count above 1.5x the mean) keep the
    split and the LSE merge.  The choice is read from the workspace's last 16 bytes, and
    the result is checked against the fp32 torch reference and against num_splits=1."""
    _print_case(test="attention_ragged_unsplit", even=even)
    past_tok, Lq, Hq, Hkv = [64 * 16, 64 * 32, 64 * 64, 64 * 128], 768, 16, 2
    B, qb = len(past_tok), Lq // 64
    ch = make_chunk(past_tok, Lq, Hq, Hkv, seed=47 + even)
    cap, P = ch.kv_cap, ch.past_blocks
    assert ops.attn_pick_splits(P, Lq, Hq, Hkv, cap) > 1
    if even:  # 16 past blocks on every row
        g = torch.Generator().manual_seed(48)
        keep_kv = torch.zeros((B, Hkv, cap), dtype=torch.uint8)
        for b in range(B):
            for h in range(Hkv):
                keep_kv[b, h, torch.randperm(P[b], generator=g)[:16]] = 1
        table, counts = ops.compact_keep_kv(keep_kv.to(gpu), P, Lq, Hq, cap)
    else:
        table, counts = ops.dense_table(P, Lq, Hq, Hkv, cap, gpu)
    cnt = counts.cpu()
    assert (2 * int(cnt.max()) * B * Hkv <= 3 * int(cnt.sum())) == even
    qg, kg, vg = ch.q.to(gpu), ch.k.to(gpu), ch.v.to(gpu)
    K, V = ops.KV.heads_first(kg), ops.KV.heads_first(vg)
    scale = 1.0 / math.sqrt(128)
    need = ops.attn_workspace_bytes(P, Lq, Hq, Hkv, cap)
    ws = torch.full((need,), 0x7F, dtype=torch.uint8, device=gpu)
    out, lse = ops.attn_fwd(qg, K, V, table, counts, P, scale, cap, Hkv, with_lse=True, workspace=ws)
    torch.cuda.synchronize()
    assert int(ws[need - 16:need - 12].cpu().view(torch.int32)[0]) == int(even)
    torch_reference_check(out, qg, kg, vg, P, table, counts, scale, lse=lse)
    one = ops.attn_fwd(qg, K, V, table, counts, P, scale, cap, Hkv, num_splits=1)
    err = (out.float() - one.float()).abs()
    assert err.max().item() <= ATOL_MAX and err.mean().item() <= ATOL_MEAN


@pytest.mark.parametrize("splits", [1, 2])
def test_attention_large_logits(gpu, splits):
    """Scores up to ~45 in log2 units (a shared direction in every query of a head and an
    offset per key block, as long-context models show): the softmax must take the scale
    in fp32 on the MFMA's fp32 scores.  Rounding q * scale * log2(e) to bf16 before the
    product instead gives each score a relative error of 2^-9, which at these magnitudes
    moves the output by ~3e-2, past the tolerance."""
    _print_case(test="attention_large_logits", splits=splits)
    B, Hq, Hkv, Lq, P = 1, 8, 2, 256, 40
    cap = P + Lq // 64
    g = torch.Generator().manual_seed(57)
    q = (torch.randn((B, Lq, Hq, 128), generator=g) + 3 * torch.randn((B, 1, Hq, 128), generator=g))
    offs = 2 * torch.randn((B, Hkv, cap, 1, 128), generator=g).expand(B, Hkv, cap, 64, 128)
    k = torch.randn((B, Hkv, cap * 64, 128), generator=g) + offs.reshape(B, Hkv, cap * 64, 128)
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    v = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    s = (q.double()[0, :, 0] @ k.double()[0, 0].T) * scale * math.log2(math.e)
    assert s.abs().max() > 30  # the regime this test is for
    keep_kv = (torch.rand((B, Hkv, cap), generator=g) < 0.5).to(torch.uint8)
    table, counts = ops.compact_keep_kv(keep_kv.to(gpu), [P], Lq, Hq, cap)
    K, V = ops.KV.heads_first(k.to(gpu)), ops.KV.heads_first(v.to(gpu))
    out = ops.attn_fwd(q.to(gpu), K, V, table, counts, [P], scale, cap, Hkv, num_splits=splits)
    torch.cuda.synchronize()
    ref = oracle.attention(bits(q), bits(k), bits(v), [P], table.cpu().numpy(), counts.cpu().numpy(), scale)
    err = np.abs(f32(out) - ref)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())
    # the decode kernel on the same inputs: the chunk's last 5 rows over the whole cache
    kv_len = [cap * 64]
    q5 = q[:, -5:].contiguous()
    dec = ops.attn_decode(q5.to(gpu), K, V, kv_len, scale, cap, Hkv, num_splits=splits)
    torch.cuda.synchronize()
    dref = oracle.attention_decode(bits(q5), bits(k), bits(v), kv_len, scale)
    err = np.abs(f32(dec) - dref)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())


def test_attention_all_selected_equals_dense(gpu):
    """Keeping every block reduces to dense causal attention (checked against torch fp32 SDPA)."""
    _print_case(test="attention_dense")
    past_tok, Lq, Hq, Hkv = 64 * 12, 128, 4, 2
    ch = make_chunk([past_tok], Lq, Hq, Hkv, seed=5, planted_blocks=0)
    table, counts = ops.dense_table(ch.past_blocks, Lq, Hq, Hkv, ch.kv_cap, gpu)
    out = ops.attn_fwd(ch.q.to(gpu), ops.KV.heads_first(ch.k.to(gpu)), ops.KV.heads_first(ch.v.to(gpu)),
                       table, counts, ch.past_blocks, 1 / math.sqrt(128), ch.kv_cap, Hkv)
    K = past_tok + Lq
    q = ch.q.float().permute(0, 2, 1, 3)  # [1, Hq, Lq, D]
    k = ch.k[:, :, :K].float().repeat_interleave(Hq // Hkv, dim=1)
    v = ch.v[:, :, :K].float().repeat_interleave(Hq // Hkv, dim=1)
    mask = torch.arange(K)[None, :] <= (past_tok + torch.arange(Lq))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask).permute(0, 2, 1, 3)
    err = (out.float().cpu() - ref).abs()
    assert err.max().item() <= ATOL_MAX and err.mean().item() <= ATOL_MEAN


# ----------------------------------------------------------------------------- decode
def test_attention_max_batch(gpu):
    """CA_MAX_BATCH (64) requests of ragged lengths (0-16 past blocks) in one launch, 2 KV
    heads each (128 KV rows), under the automatic plan, against the fp64 oracle."""
    _print_case(test="attention_max_batch")
    g = torch.Generator().manual_seed(95)
    past = [64 * int(x) for x in torch.randint(0, 17, (64,), generator=g)]
    _attn_case(gpu, past, 64, 4, 2, "heads_first", 0, 0.4, seed=95)


def test_attention_more_kv_rows_than_the_placement_table(gpu):
    """36 requests x 16 KV heads = 576 KV rows, more than the 512 placement units the plan
    holds: work items are decoded by request offsets instead of per-XCD units (automatic
    plan and a forced split count), against the fp64 oracle."""
    g = torch.Generator().manual_seed(96)
    past = [64 * int(x) for x in torch.randint(0, 17, (36,), generator=g)]
    for splits in (0, 2):
        _print_case(test="attention_576_rows", splits=splits)
        _attn_case(gpu, past, 64, 16, 16, "heads_first", splits, 0.4, seed=96)


def _decode_case(gpu, kv_len, Lq, Hq, Hkv, layout, splits, seed, with_prefill_check=False):
    """Dense decode over each request's whole cache against the fp64 oracle.  Cache slots
    past kv_len hold NaN: the kernel must neither read them into the result nor let them
    meet zero weights."""
    B = len(kv_len)
    cap = (max(kv_len) + 63) // 64
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, Lq, Hq, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16)
    for b, n in enumerate(kv_len):
        k[b, :, n:] = float("nan")
        v[b, :, n:] = float("nan")
    qg = q.to(gpu)
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
    out, lse = ops.attn_decode(qg, K, V, kv_len, scale, cap, Hkv, with_lse=True, num_splits=splits)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.attention_decode(bits(q), bits(k), bits(v), kv_len, scale, with_lse=True)
    got = f32(out)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert err.max() <= ATOL_MAX, err.max()
    assert err.mean() <= ATOL_MEAN, err.mean()
    lerr = np.abs(f32(lse) - ref_lse)
    assert lerr.max() <= 4e-3, lerr.max()
    return out


@pytest.mark.parametrize("splits", [0, 1, 5])
@pytest.mark.parametrize("layout", ["heads_first", "seq_first", "paged"])
def test_decode_layouts_and_splits(gpu, layout, splits):
    _print_case(test="decode", layout=layout, splits=splits)
    _decode_case(gpu, [1, 777, 64 * 40 + 13], 1, 8, 2, layout, splits, seed=51)


@pytest.mark.parametrize("G,Lq", [(1, 1), (4, 3), (7, 5), (8, 64), (16, 1)])
def test_decode_groups_and_query_rows(gpu, G, Lq):
    _print_case(test="decode_groups", G=G, Lq=Lq)
    _decode_case(gpu, [Lq, 64 * 9 + 7, 1000], Lq, 2 * G, 2, "heads_first", 0, seed=60 + G)


def test_decode_max_batch_many_rows(gpu):
    """CA_MAX_BATCH (64) requests x 16 KV heads = 1024 KV rows (more than the plan's 512
    placement units), ragged unaligned lengths, automatic and forced splits, against the
    fp64 decode oracle."""
    g = torch.Generator().manual_seed(97)
    kv = [int(x) for x in torch.randint(1, 1000, (64,), generator=g)]
    for splits in (0, 3):
        _print_case(test="decode_1024_rows", splits=splits)
        _decode_case(gpu, kv, 1, 16, 16, "heads_first", splits, seed=97)


def test_decode_long_context_plan(gpu):
    """A 32K-token request beside a short one: the plan splits the long rows (at least 4
    blocks per split, at most 32 splits), so the result goes through the LSE merge."""
    _print_case(test="decode_long")
    kv = [64 * 512 + 1, 5000]
    cap = (max(kv) + 63) // 64
    assert ops.attn_decode_workspace_bytes(kv, 1, 32, 8, cap, 0) >= ops.attn_decode_workspace_bytes(kv, 1, 32, 8, cap,
                                                                                                     16)
    _decode_case(gpu, kv, 1, 32, 8, "heads_first", 0, seed=71)


def test_decode_equals_prefill_on_aligned_shapes(gpu):
    """On 64-aligned shapes decode is dense prefill of the last chunk: with one split each,
    both entry points run the same blocks in the same order and agree bit for bit."""
    _print_case(test="decode_vs_prefill")
    past, Lq, Hq, Hkv = [7, 0, 3], 64, 8, 2
    B, cap = len(past), max(past) + 1
    g = torch.Generator().manual_seed(81)
    q = torch.randn((B, Lq, Hq, 128), generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn((B, Hkv, cap * 64, 128), generator=g).to(torch.bfloat16).to(gpu)
    K, V = ops.KV.heads_first(k), ops.KV.heads_first(v)
    table, counts = ops.dense_table(past, Lq, Hq, Hkv, cap, gpu)
    scale = 1.0 / math.sqrt(128)
    pre, pre_lse = ops.attn_fwd(q, K, V, table, counts, past, scale, cap, Hkv, with_lse=True, num_splits=1)
    dec, dec_lse = ops.attn_decode(q, K, V, [64 * (p + 1) for p in past], scale, cap, Hkv, with_lse=True,
                                   num_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(pre.view(torch.int16), dec.view(torch.int16))
    assert torch.equal(pre_lse, dec_lse)


def test_decode_cache_ending_at_kv_len(gpu):
    """The decode kernel's reads stop at kv_len (the partial last block's buffer range ends
    there), so a contiguous cache holding exactly kv_len tokens is valid; one token short is
    refused on the host."""
    _print_case(test="decode_exact_cache")
    g = torch.Generator().manual_seed(23)
    q = torch.randn((1, 3, 4, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 2, 100, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, 2, 100, 128), generator=g).to(torch.bfloat16)
    K, V = ops.KV.heads_first(k.to(gpu)), ops.KV.heads_first(v.to(gpu))
    out = ops.attn_decode(q.to(gpu), K, V, [100], 0.1, 2, 2)
    ref = oracle.attention_decode(bits(q), bits(k), bits(v), [100], 0.1)
    err = np.abs(f32(out) - ref)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())
    with pytest.raises(ValueError, match="holds 100 tokens"):
        ops.attn_decode(q.to(gpu), K, V, [101], 0.1, 2, 2)


def test_host_checks_cover_kv_rows_and_out(gpu):
    """Caches with fewer requests or KV heads than the call addresses, and outputs of another
    shape, are refused on the host before any launch."""
    _print_case(test="host_checks")
    q = torch.zeros((2, 64, 4, 128), dtype=torch.bfloat16, device=gpu)
    kc = torch.zeros((1, 2, 128, 128), dtype=torch.bfloat16, device=gpu)
    K = ops.KV.heads_first(kc)
    table, counts = ops.dense_table([1, 1], 64, 4, 2, 2, gpu)
    with pytest.raises(ValueError, match="1 requests x 2 KV heads"):
        ops.attn_fwd(q, K, K, table, counts, [1, 1], 0.1, 2, 2)
    with pytest.raises(ValueError, match="1 requests x 2 KV heads"):
        ops.attn_decode(q[:, :1], K, K, [100, 100], 0.1, 2, 2)
    kc2 = torch.zeros((2, 128, 1, 128), dtype=torch.bfloat16, device=gpu)  # seq-first, one head
    with pytest.raises(ValueError, match="2 requests x 1 KV heads"):
        ops.attn_fwd(q, ops.KV.seq_first(kc2), ops.KV.seq_first(kc2), table, counts, [1, 1], 0.1, 2, 2)
    kn = torch.zeros((2, 64, 2, 128), dtype=torch.bfloat16, device=gpu)
    kmean = torch.zeros((4, 2, 128), dtype=torch.float32, device=gpu)
    with pytest.raises(ValueError, match="1 requests x 2 KV heads"):
        ops.cache_fill(kn, kn, K, K, [1, 1], 2, kmean)
    kb = torch.zeros((2, 2, 128, 128), dtype=torch.bfloat16, device=gpu)
    KB = ops.KV.heads_first(kb)
    with pytest.raises(ValueError, match="must have q's shape"):
        ops.attn_fwd(q, KB, KB, table, counts, [1, 1], 0.1, 2, 2, out=q[:, :, :2])
    with pytest.raises(ValueError, match="must have q's shape"):
        ops.attn_decode(q[:, :1], KB, KB, [100, 100], 0.1, 2, 2, out=q[:1, :1])
    with pytest.raises(ValueError, match="1 per-request values for a batch of 2"):
        ops.attn_fwd(q, KB, KB, table, counts, [1], 0.1, 2, 2)
    rowmask = torch.zeros((2, 4, 1, 2), dtype=torch.int32, device=gpu)  # words_for(2) is 1
    with pytest.raises(ValueError, match="rowmask must be contiguous"):
        ops.union_compact(rowmask, [1, 1], 2, 2)
    torch.cuda.synchronize()
