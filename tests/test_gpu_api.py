"""GPU parity of the reference-shaped operator API against the CPU oracle.

Each test drives one public entry point the way the reference's callers do and checks
the result against the oracle: selections/tables/summaries bit-exact, attention output
within the north-star tolerance (max-abs 2e-2, mean-abs 2e-3).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from compactattention_amd import ops
from compactattention_amd.flashprefill_vendor import (flash_prefill_compute_mean_k,
                                                      flash_prefill_score_chunked_from_mean_k, mean_k_kernel_layout)
from compactattention_amd.kv_cache import PagedKVCache
from compactattention_amd.modules.attention_forward_chunked_dense import (
    chunked_prefill_column_dense_attention_forward, chunked_prefill_column_dense_attention_from_keep_block)
from compactattention_amd.modules.flashprefill_prefill import (flashprefill_compactattn_prefill_full_kv,
                                                               flashprefill_rule)
from compactattention_amd.prefill_sparse.attn_gate import AttnGate
from compactattention_amd.synthetic import make_chunk, rope_tables

from .util import bits, f32, float_bits_equal, ref_flashprefill_tables

pytestmark = pytest.mark.gpu

ATOL_MAX = 2e-2
ATOL_MEAN = 2e-3
SCALE = 1.0 / math.sqrt(128)


def _print_case(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _seq_first(t):  # heads-first [B, Hkv, K, D] -> [B, K, Hkv, D]
    return t.transpose(1, 2).contiguous()


def _check_attention(out, ch, table, counts):
    ref = oracle.attention(bits(ch.q), bits(ch.k), bits(ch.v), ch.past_blocks, table, counts, SCALE)
    err = np.abs(f32(out) - ref)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())


@pytest.mark.parametrize("kv_group_aware", [False, True])
@pytest.mark.parametrize("use_hf", [False, True])
def test_seer_forward_threshold(gpu, use_hf, kv_group_aware):
    _print_case(test="seer_forward", use_hf=use_hf, kv_group_aware=kv_group_aware)
    Hq, Hkv, Lq, past = 8, 2, 256, 64 * 30
    ch = make_chunk([past], Lq, Hq, Hkv, seed=3)
    P, cap = ch.past_blocks, ch.kv_cap
    Hs = Hkv if kv_group_aware else Hq
    g = torch.Generator().manual_seed(9)
    logits = torch.randn((1, Hs, Lq // 64, cap), generator=g) * 2
    causal = torch.arange(cap)[None, :] <= (P[0] + torch.arange(Lq // 64))[:, None]
    gate = torch.softmax(logits.masked_fill(~causal, float("-inf")), dim=-1)
    thr = 0.02
    kw = dict(k_hf=ch.k.to(gpu), v_hf=ch.v.to(gpu)) if use_hf else {}
    out, stats = chunked_prefill_column_dense_attention_forward(
        ch.q.to(gpu), _seq_first(ch.k).to(gpu), _seq_first(ch.v).to(gpu), None, Lq, softmax_scale=SCALE,
        attn_gate_score=gate.to(gpu), threshold=thr, num_key_value_groups=Hq // Hkv,
        attn_gate_is_kv_group_aware=kv_group_aware, pack_impl="indexed_dense", indexed_impl="fi_zero_copy",
        return_stats=True, **kw)
    keep = oracle.select_rows(gate.numpy(), P, oracle.Rule(threshold=thr))
    _, _, table, counts = oracle.union_compact(keep, Hkv, P)
    assert stats["col_selected_blocks"] == counts.sum()
    _check_attention(out, ch, table, counts)


def test_from_keep_block_matches_union(gpu):
    _print_case(test="from_keep_block")
    Hq, Hkv, Lq, past = 8, 2, 128, 64 * 17
    ch = make_chunk([past], Lq, Hq, Hkv, seed=4)
    cap = ch.kv_cap
    g = torch.Generator().manual_seed(1)
    keep_block = torch.rand((1, Hq, cap), generator=g) < 0.3
    out, _ = chunked_prefill_column_dense_attention_from_keep_block(
        ch.q.to(gpu), _seq_first(ch.k).to(gpu), _seq_first(ch.v).to(gpu), keep_block.to(gpu), None, Lq, SCALE,
        num_key_value_groups=Hq // Hkv)
    kv = keep_block.view(1, Hkv, Hq // Hkv, cap).any(dim=2).numpy().astype(np.uint8)
    kv[..., ch.past_blocks[0]:] = 1
    table = np.full((Hkv, cap), -1, np.int32)
    counts = np.zeros((Hkv,), np.int32)
    for h in range(Hkv):
        ids = np.nonzero(kv[0, h])[0]
        table[h, :len(ids)] = ids
        counts[h] = len(ids)
    _check_attention(out, ch, table, counts)


@pytest.mark.parametrize("params", [
    dict(attention_sink=2, window_size=4, alpha=0.06, last_n_block=2, min_budget=0),
    dict(attention_sink=1, window_size=0, alpha=0.5, last_n_block=0, min_budget=6),
    dict(attention_sink=2, window_size=4, alpha=0.06, last_n_block=1, min_budget=12),
    dict(attention_sink=0, window_size=2, alpha=0.9, last_n_block=0, min_budget=30),
])
def test_flashprefill_entry(gpu, params):
    """The entry's tables (through the rule it builds, flashprefill_rule) and its output
    against the reference's selection semantics: a torch restatement of
    _flashprefill_keep_block_from_scores_rowwise (flashprefill_prefill.py:596-666, min_budget
    by torch.topk over all Kb columns of the zeroed row) applied to the fp32 scores, which
    the GPU reproduces bit for bit.  The scores are continuous, so the only ties are the
    zeroed non-causal columns, which the causal mask drops whichever torch.topk picks."""
    _print_case(test="flashprefill_entry", **params)
    Hq, Hkv, Lq, past = 8, 2, 256, 64 * 40
    ch = make_chunk([past], Lq, Hq, Hkv, seed=5)
    P, cap = ch.past_blocks, ch.kv_cap
    ks = _seq_first(ch.k).to(gpu)
    mean_k = flash_prefill_compute_mean_k(ks, block_size=64)
    out, _ = flashprefill_compactattn_prefill_full_kv(
        ch.q.to(gpu), ks, _seq_first(ch.v).to(gpu), None, softmax_scale=SCALE, num_key_value_groups=Hq // Hkv,
        block_size=64, pack_impl="indexed_dense", indexed_impl="fi_zero_copy", cache_fill_backend="cuda",
        mean_k_cache=mean_k, **params)
    khat = oracle.block_mean(bits(_seq_first(ch.k)))
    qhat = oracle.block_mean(bits(ch.q))
    sc = oracle.block_scores(qhat, khat, P, SCALE)
    ref_table, ref_counts = ref_flashprefill_tables(sc, P, Hkv, params["alpha"], params["attention_sink"],
                                                    params["window_size"], params["min_budget"],
                                                    params["last_n_block"])
    # the oracle's all-columns rule is the same selection
    rule = oracle.Rule(topk=params["min_budget"], alpha=params["alpha"], sink_blocks=params["attention_sink"],
                       window_blocks=params["window_size"], last_n_block=params["last_n_block"],
                       topk_all_columns=True)
    _, _, table, counts = oracle.union_compact(oracle.select_rows(sc, P, rule), Hkv, P, params["last_n_block"])
    assert np.array_equal(counts, ref_counts) and np.array_equal(table, ref_table)
    # the GPU tables through the entry's own rule
    gqhat = ops.pool_query(ch.q.to(gpu), P, cap, num_kv_heads=Hkv)
    grule = flashprefill_rule(params["attention_sink"], params["window_size"], params["alpha"],
                              params["last_n_block"], params["min_budget"])
    rowmask, _ = ops.score_select(gqhat, mean_k_kernel_layout(mean_k), SCALE, grule, P, Hkv, cap)
    gtable, gcounts, _, _ = ops.union_compact(rowmask, P, Hkv, cap, last_n_block=params["last_n_block"])
    assert np.array_equal(gcounts.cpu().numpy(), ref_counts)
    assert np.array_equal(gtable.cpu().numpy(), ref_table)
    _check_attention(out, ch, ref_table, ref_counts)


def test_flashprefill_first_chunk_is_dense(gpu):
    _print_case(test="flashprefill_first_chunk")
    ch = make_chunk([0], 128, 4, 2, seed=6)
    out, stats = flashprefill_compactattn_prefill_full_kv(
        ch.q.to(gpu), _seq_first(ch.k).to(gpu), _seq_first(ch.v).to(gpu), None, softmax_scale=SCALE,
        num_key_value_groups=2, block_size=64, attention_sink=2, window_size=4, alpha=0.06, last_n_block=0,
        min_budget=0, pack_impl="indexed_dense", indexed_impl="fi_zero_copy", cache_fill_backend="auto")
    assert stats["flashprefill_dense_calls"] == 1.0
    table = np.tile(np.arange(ch.kv_cap, dtype=np.int32), (2, 1))
    _check_attention(out, ch, table, np.full((2,), ch.kv_cap, np.int32))


def test_flashprefill_scores_bit_exact(gpu):
    _print_case(test="flashprefill_scores")
    ch = make_chunk([64 * 21], 192, 6, 3, seed=7)
    ks = _seq_first(ch.k).to(gpu)
    mean_k = flash_prefill_compute_mean_k(ks, block_size=64)
    khat = oracle.block_mean(bits(_seq_first(ch.k)))
    assert float_bits_equal(f32(mean_k.permute(0, 2, 1, 3)), khat)
    sc = flash_prefill_score_chunked_from_mean_k(ch.q.to(gpu), mean_k, key_len=ks.shape[1], block_size=64)
    ref = oracle.block_scores(oracle.block_mean(bits(ch.q)), khat, ch.past_blocks, SCALE)
    assert float_bits_equal(f32(sc.permute(0, 3, 1, 2)), ref)


def test_attn_gate_bit_exact(gpu):
    _print_case(test="attn_gate")
    Hq, Hkv, Lq, past = 8, 2, 128, 64 * 12
    ch = make_chunk([past], Lq, Hq, Hkv, seed=8)
    gate = AttnGate(64, 128, 128, Hkv, Hq).to(gpu)
    gate.reset_parameters(0.02, torch.Generator().manual_seed(2))
    cos, sin = rope_tables(ch.kv_cap)
    scores = gate(ch.q.to(gpu), _seq_first(ch.k).to(gpu), position_embeddings=(cos.to(gpu), sin.to(gpu)))
    wq = f32(gate.mask_linear_q.weight)
    wk = f32(gate.mask_linear_k.weight)
    P = ch.past_blocks
    qg = oracle.gate_project(oracle.block_mean(bits(ch.q)), wq, f32(cos), f32(sin), P)
    kg = oracle.gate_project(oracle.block_mean(bits(_seq_first(ch.k))), wk, f32(cos), f32(sin), [0])
    ref = oracle.block_scores(qg, kg, P, 128 ** -0.5)
    assert float_bits_equal(f32(scores), ref)


def test_paged_cache_appends(gpu):
    _print_case(test="paged_cache")
    Hkv = 2
    cache = PagedKVCache(1, Hkv, 64 * 20, gpu, with_kmean=True, with_kgate=True)
    g = torch.Generator().manual_seed(12)
    chunks = [torch.randn((1, 64 * n, Hkv, 128), generator=g).to(torch.bfloat16) for n in (5, 3, 4)]
    vals = [torch.randn_like(c.float()).to(torch.bfloat16) for c in chunks]
    wk = (torch.randn((Hkv, 128, 128), generator=g) * 0.02).float()
    cos, sin = rope_tables(20)
    for c, v in zip(chunks, vals):
        cache.append(c.to(gpu), v.to(gpu), gate_wk=wk.to(gpu), rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
    allk = torch.cat(chunks, dim=1)
    allv = torch.cat(vals, dim=1)
    assert cache.length == allk.shape[1]
    assert torch.equal(cache.k_hf().cpu(), allk.transpose(1, 2))
    assert torch.equal(cache.v_hf().cpu(), allv.transpose(1, 2))
    means = oracle.block_mean(bits(allk))
    nb = allk.shape[1] // 64
    assert float_bits_equal(f32(cache.kmean[:, :, :nb]), means)
    assert float_bits_equal(f32(cache.kgate[:, :, :nb]), oracle.gate_project(means, f32(wk), f32(cos), f32(sin), [0]))
