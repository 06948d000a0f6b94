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
from compactattention_amd.prefill_sparse.attn_gate import ATTNGATE_CLASSES
from compactattention_amd.synthetic import make_chunk, rope_tables

from .util import (bits, f32, float_bits_equal, oracle_gate_summaries, ref_flashprefill_tables, ref_seer_tables,
                   spy_union_compact, torch_reference_check)

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


@pytest.mark.parametrize("Qb,keep_recent", [(1, 2), (1, 4), (16, 2), (16, 4), (4, 9)])
@pytest.mark.parametrize("kv_group_aware", [False, True])
def test_seer_entry_reference_rule(gpu, monkeypatch, Qb, keep_recent, kv_group_aware):
    """The Seer entry's tables equal the reference's selection (a torch restatement of
    _build_keep_block_mask_chunked_fast_path + _build_kv_head_union_keep_block_mask,
    attention_forward_chunked_dense.py:559-683) bit for bit: strict threshold over the query
    blocks, the last keep_recent_blocks KV columns forced -- past blocks too once
    keep_recent_blocks exceeds the chunk's Qb blocks -- and the GQA union; then every query row
    of the output against an fp32 torch attention over those tables."""
    _print_case(test="seer_entry_reference_rule", Qb=Qb, keep_recent=keep_recent, kv_group_aware=kv_group_aware)
    Hq, Hkv, Lq, past = 8, 2, 64 * Qb, 64 * 44
    ch = make_chunk([past, past], Lq, Hq, Hkv, seed=30 + Qb)
    P, cap = ch.past_blocks, ch.kv_cap
    Hs = Hkv if kv_group_aware else Hq
    g = torch.Generator().manual_seed(31)
    logits = torch.randn((2, Hs, Qb, cap), generator=g) * 2.5
    causal = torch.arange(cap)[None, :] <= (P[0] + torch.arange(Qb))[:, None]
    gate = torch.softmax(logits.masked_fill(~causal, float("-inf")), dim=-1)
    thr = 0.03
    calls = spy_union_compact(monkeypatch)
    out, stats = chunked_prefill_column_dense_attention_forward(
        ch.q.to(gpu), _seq_first(ch.k).to(gpu), _seq_first(ch.v).to(gpu), None, Lq, softmax_scale=SCALE,
        attn_gate_score=gate.to(gpu), threshold=thr, keep_recent_blocks=keep_recent, num_key_value_groups=Hq // Hkv,
        attn_gate_is_kv_group_aware=kv_group_aware, pack_impl="indexed_dense", return_stats=True,
        k_hf=ch.k.to(gpu), v_hf=ch.v.to(gpu))
    ref_table, ref_counts = ref_seer_tables(gate.numpy(), P, Hkv, thr, keep_recent, kv_group_aware=kv_group_aware)
    assert len(calls) == 1
    table, counts = (t.cpu().numpy() for t in calls[0])
    assert np.array_equal(counts, ref_counts)
    assert np.array_equal(table, ref_table)
    assert stats["col_selected_blocks"] == ref_counts.sum()
    assert ref_counts.min() < P[0] + Qb, "the case should drop blocks"
    if keep_recent > Qb:  # the forced past blocks right before the chunk
        for r in range(2 * Hkv):
            assert set(range(P[0] - (keep_recent - Qb), P[0])) <= set(ref_table[r, :ref_counts[r]].tolist())
    torch_reference_check(out, ch.q.to(gpu), ch.k.to(gpu), ch.v.to(gpu), P, calls[0][0], calls[0][1], SCALE)


def test_seer_entry_per_request_threshold(gpu, monkeypatch):
    """A 1-D threshold tensor selects each request with its own value (the reference's
    view(-1, 1, 1) broadcast, attention_forward_chunked_dense.py:383-393); the tables equal the
    restatement with per-request thresholds, and request 1's equal a scalar call's with its value."""
    _print_case(test="seer_entry_per_request_threshold")
    Hq, Hkv, Lq, past = 8, 2, 256, 64 * 30
    ch = make_chunk([past, past], Lq, Hq, Hkv, seed=41)
    P, cap = ch.past_blocks, ch.kv_cap
    g = torch.Generator().manual_seed(42)
    logits = torch.randn((2, Hq, Lq // 64, cap), generator=g) * 2.5
    causal = torch.arange(cap)[None, :] <= (P[0] + torch.arange(Lq // 64))[:, None]
    gate = torch.softmax(logits.masked_fill(~causal, float("-inf")), dim=-1)
    thr = torch.tensor([0.01, 0.08])
    calls = spy_union_compact(monkeypatch)
    args = (ch.q.to(gpu), _seq_first(ch.k).to(gpu), _seq_first(ch.v).to(gpu), None, Lq)
    kw = dict(softmax_scale=SCALE, attn_gate_score=gate.to(gpu), num_key_value_groups=Hq // Hkv)
    chunked_prefill_column_dense_attention_forward(*args, threshold=thr.to(gpu), **kw)
    ref_table, ref_counts = ref_seer_tables(gate.numpy(), P, Hkv, thr.tolist(), 2)
    table, counts = (t.cpu().numpy() for t in calls[0])
    assert np.array_equal(counts, ref_counts) and np.array_equal(table, ref_table)
    assert ref_counts[:Hkv].sum() > ref_counts[Hkv:].sum()  # the lower threshold keeps more
    chunked_prefill_column_dense_attention_forward(*args, threshold=0.08, **kw)
    assert np.array_equal(calls[1][0].cpu().numpy()[Hkv:], table[Hkv:])
    with pytest.raises(ValueError, match="threshold tensor has 3 values"):
        chunked_prefill_column_dense_attention_forward(*args, threshold=torch.tensor([0.1, 0.2, 0.3]), **kw)
    with pytest.raises(ValueError, match="Expected scalar or 1D"):
        chunked_prefill_column_dense_attention_forward(*args, threshold=torch.ones((2, 1)), **kw)


def test_seer_entry_short_gate_scores(gpu, monkeypatch):
    """Gate scores over only the last key blocks (the reference right-aligns such a short keep
    mask, _project_short_qhead_keep_block_to_kv_full_width, :708-734): the leading columns are
    never selected, the covered ones follow the rule."""
    _print_case(test="seer_entry_short_gate")
    Hq, Hkv, Lq, past = 4, 2, 128, 64 * 20
    ch = make_chunk([past], Lq, Hq, Hkv, seed=43)
    P, cap = ch.past_blocks, ch.kv_cap
    short = 12
    g = torch.Generator().manual_seed(44)
    gate_short = torch.rand((1, Hq, Lq // 64, short), generator=g) * 0.1
    calls = spy_union_compact(monkeypatch)
    chunked_prefill_column_dense_attention_forward(
        ch.q.to(gpu), _seq_first(ch.k).to(gpu), _seq_first(ch.v).to(gpu), None, Lq, softmax_scale=SCALE,
        attn_gate_score=gate_short.to(gpu), threshold=0.06, keep_recent_blocks=5, num_key_value_groups=Hq // Hkv)
    full = torch.zeros((1, Hq, Lq // 64, cap))
    full[..., cap - short:] = gate_short
    ref_table, ref_counts = ref_seer_tables(full.numpy(), P, Hkv, 0.06, 5)
    table, counts = (t.cpu().numpy() for t in calls[0])
    assert np.array_equal(counts, ref_counts) and np.array_equal(table, ref_table)
    assert all(ref_table[r, 0] >= cap - short for r in range(Hkv))


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


def _pad_keys(x, cap):
    """[B, K, H, D] -> heads-first [B, H, cap*64, D] with zero rows past K (never visible to a query)."""
    out = torch.zeros((x.shape[0], x.shape[2], cap * 64, x.shape[3]), dtype=x.dtype)
    out[:, :, :x.shape[1]] = x.transpose(1, 2)
    return out


@pytest.mark.parametrize("q_len", [37, 256 + 37])
def test_unaligned_chunk_selects_with_a_partial_block(gpu, monkeypatch, q_len):
    """A chunk of q_len tokens (not a multiple of 64) starting at a block boundary, through the
    FlashPrefill entry and both Seer entries: ceil(q_len/64) query blocks whose last pools its
    q_len % 64 tokens (as compute_mean_vector and AttnGate's ceil_mode pools do), key blocks up
    to the partial last one, the reference's selection over them, the partial current block
    kept, and every query row -- the tail queries included -- attending over the selected past
    blocks and the current chunk with the causal mask at the true positions (the reference's
    padded indexed path, attention_forward_chunked_dense.py:438-491, without its padded-length
    causal alignment).  Tables bit-exact against the oracle's; every output row against the
    fp64 oracle over those tables."""
    _print_case(test="unaligned_chunk", q_len=q_len)
    Hq, Hkv, past = 8, 2, 64 * 40
    G = Hq // Hkv
    kv_len = past + q_len
    P = [past // 64]
    Qb = -(-q_len // 64)
    cap = P[0] + Qb
    g = torch.Generator().manual_seed(q_len)
    # block structure (a shared direction per query head, an offset per key block) makes the
    # pooled scores selective
    q = (torch.randn((1, q_len, Hq, 128), generator=g) + 3 * torch.randn((1, 1, Hq, 128), generator=g))
    q = q.to(torch.bfloat16)
    offs = 2 * torch.randn((1, cap, 1, Hkv, 128), generator=g).expand(1, cap, 64, Hkv, 128).reshape(1, cap * 64, Hkv, 128)
    k = (torch.randn((1, kv_len, Hkv, 128), generator=g) + offs[:, :kv_len]).to(torch.bfloat16)
    v = torch.randn((1, kv_len, Hkv, 128), generator=g).to(torch.bfloat16)
    kp, vp = _pad_keys(k, cap), _pad_keys(v, cap)

    def check(out, table, counts):
        ref = oracle.attention(bits(q), bits(kp), bits(vp), P, table, counts, SCALE)
        err = np.abs(f32(out) - ref)
        assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())
        assert (counts < cap).any(), "the case should drop blocks"

    calls = spy_union_compact(monkeypatch)

    def no_dense(*args, **kw):  # no query of the chunk takes the dense decode path
        raise AssertionError("an aligned-start chunk must not attend densely")

    monkeypatch.setattr(ops, "attn_decode", no_dense)
    # FlashPrefill: pooled scores over the partial blocks, the reference's rowwise rule
    fp = dict(attention_sink=1, window_size=2, alpha=0.5, last_n_block=0, min_budget=3)
    out, _ = flashprefill_compactattn_prefill_full_kv(
        q.to(gpu), k.to(gpu), v.to(gpu), None, softmax_scale=SCALE, num_key_value_groups=G, block_size=64,
        pack_impl="indexed_dense", indexed_impl="fi_zero_copy", cache_fill_backend="auto", **fp)
    sc = oracle.block_scores(oracle.block_mean(bits(q)), oracle.block_mean(bits(k)), P, SCALE)
    assert sc.shape[2:] == (Qb, cap)
    table, counts = ref_flashprefill_tables(sc, P, Hkv, fp["alpha"], fp["attention_sink"], fp["window_size"],
                                            fp["min_budget"], fp["last_n_block"])
    gt, gc = (t.cpu().numpy() for t in calls[-1])
    assert np.array_equal(gc, counts) and np.array_equal(gt, table)
    check(out, table, counts)
    # Seer: threshold on caller gate scores over ceil(q_len/64) x ceil(kv_len/64) blocks
    logits = torch.randn((1, Hq, Qb, cap), generator=g) * 2.5
    causal = torch.arange(cap)[None, :] <= (P[0] + torch.arange(Qb))[:, None]
    gate = torch.softmax(logits.masked_fill(~causal, float("-inf")), dim=-1)
    out, _ = chunked_prefill_column_dense_attention_forward(
        q.to(gpu), k.to(gpu), v.to(gpu), None, q_len, softmax_scale=SCALE, attn_gate_score=gate.to(gpu),
        threshold=0.05, num_key_value_groups=G, pack_impl="indexed_dense", indexed_impl="fi_zero_copy")
    table, counts = ref_seer_tables(gate.numpy(), P, Hkv, 0.05, 2)
    gt, gc = (t.cpu().numpy() for t in calls[-1])
    assert np.array_equal(gc, counts) and np.array_equal(gt, table)
    check(out, table, counts)
    # caller keep masks over ceil(kv_len/64) blocks
    keep_block = torch.rand((1, Hq, cap), generator=g) < 0.2
    out, _ = chunked_prefill_column_dense_attention_from_keep_block(
        q.to(gpu), k.to(gpu), v.to(gpu), keep_block.to(gpu), None, q_len, SCALE, num_key_value_groups=G)
    kv = keep_block.view(1, Hkv, G, cap).any(dim=2).numpy().astype(np.uint8)
    kv[..., P[0]:] = 1
    table = np.full((Hkv, cap), -1, np.int32)
    counts = np.zeros((Hkv,), np.int32)
    for h in range(Hkv):
        ids = np.nonzero(kv[0, h])[0]
        table[h, :len(ids)] = ids
        counts[h] = len(ids)
    check(out, table, counts)


@pytest.mark.parametrize("q_len", [1, 5, 64])
def test_mid_block_and_single_token_calls_are_dense(gpu, q_len):
    """q_len == 1 (FlashPrefill's dense fallback, flashprefill_prefill.py:903-907) and chunks of
    at most 64 queries that start inside a block attend densely to all kv_len keys; a longer
    chunk that starts inside a block raises."""
    _print_case(test="mid_block_dense", q_len=q_len)
    Hq, Hkv = 4, 2
    kv_len = 64 * 9 + 20 + q_len  # the chunk starts 20 tokens into block 9
    g = torch.Generator().manual_seed(100 + q_len)
    q = torch.randn((1, q_len, Hq, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, kv_len, Hkv, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, kv_len, Hkv, 128), generator=g).to(torch.bfloat16)
    ref = oracle.attention_decode(bits(q), bits(k.transpose(1, 2)), bits(v.transpose(1, 2)), [kv_len], SCALE)
    fp = dict(attention_sink=1, window_size=2, alpha=0.3, last_n_block=0, min_budget=4, pack_impl="indexed_dense",
              indexed_impl="fa2_paged", cache_fill_backend="auto")
    out, stats = flashprefill_compactattn_prefill_full_kv(q.to(gpu), k.to(gpu), v.to(gpu), None, softmax_scale=SCALE,
                                                          num_key_value_groups=2, block_size=64, **fp)
    assert stats["flashprefill_dense_calls"] == 1.0
    err = np.abs(f32(out) - ref)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN
    if q_len > 1:
        gate = torch.rand((1, Hq, 2, -(-kv_len // 64)), generator=g)
        out, _ = chunked_prefill_column_dense_attention_forward(
            q.to(gpu), k.to(gpu), v.to(gpu), None, q_len, softmax_scale=SCALE, attn_gate_score=gate.to(gpu),
            threshold=0.5, num_key_value_groups=2)
        err = np.abs(f32(out) - ref)
        assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN
    long_q = torch.zeros((1, 65, Hq, 128), dtype=torch.bfloat16)
    kk = torch.zeros((1, 64 * 3 + 10 + 65, Hkv, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="block boundary"):
        flashprefill_compactattn_prefill_full_kv(long_q.to(gpu), kk.to(gpu), kk.to(gpu), None, softmax_scale=SCALE,
                                                 num_key_value_groups=2, block_size=64, **fp)


@pytest.mark.parametrize("q_len", [256, 256 + 64, 256 + 37])
def test_flashprefill_entry_128_token_blocks(gpu, monkeypatch, q_len):
    """block_size=128 (the reference's default, modeling_llama_flashprefill_compactattn.py:253):
    128-token score blocks pooled from the 64-token means, the rowwise rule in 128-token block
    units (a torch restatement of flashprefill_prefill.py:596-666 on the oracle's 128-token
    scores), then both 64-token pages of every kept 128-token block (one when the chunk's last
    128-token block has a single 64-token page).  Tables bit-exact; attention against the fp64
    oracle; flash_prefill_compute_mean_k / score_chunked at block 128 agree with the oracle."""
    _print_case(test="flashprefill_128", q_len=q_len)
    Hq, Hkv, past = 8, 2, 64 * 40
    G = Hq // Hkv
    kv_len = past + q_len
    cap64 = past // 64 + -(-q_len // 64)
    g = torch.Generator().manual_seed(7 + q_len)
    q = (torch.randn((1, q_len, Hq, 128), generator=g) + 3 * torch.randn((1, 1, Hq, 128), generator=g))
    q = q.to(torch.bfloat16)
    nb = -(-kv_len // 128)
    offs = 2 * torch.randn((1, nb, 1, Hkv, 128), generator=g).expand(1, nb, 128, Hkv, 128).reshape(1, nb * 128, Hkv, 128)
    k = (torch.randn((1, kv_len, Hkv, 128), generator=g) + offs[:, :kv_len]).to(torch.bfloat16)
    v = torch.randn((1, kv_len, Hkv, 128), generator=g).to(torch.bfloat16)
    calls = spy_union_compact(monkeypatch)
    fp = dict(attention_sink=1, window_size=2, alpha=0.4, last_n_block=1, min_budget=3)
    out, _ = flashprefill_compactattn_prefill_full_kv(
        q.to(gpu), k.to(gpu), v.to(gpu), None, softmax_scale=SCALE, num_key_value_groups=G, block_size=128,
        pack_impl="indexed_dense", indexed_impl="fa2_paged", cache_fill_backend="auto", **fp)
    m64q, m64k = oracle.block_mean(bits(q)), oracle.block_mean(bits(k))
    last = q_len - 64 * (m64q.shape[2] - 1)
    q128 = oracle.pair_block_means(m64q, last)
    k128 = oracle.pair_block_means(m64k, last)
    P128 = [past // 128]
    sc = oracle.block_scores(q128, k128, P128, SCALE)
    t128, c128 = ref_flashprefill_tables(sc, P128, Hkv, fp["alpha"], fp["attention_sink"], fp["window_size"],
                                         fp["min_budget"], fp["last_n_block"])
    # the 128-token union is the one the entry built before naming pages
    gt, gc = (t.cpu().numpy() for t in calls[-1])
    assert np.array_equal(gc, c128) and np.array_equal(gt, t128)
    table = np.full((Hkv, cap64), -1, np.int32)
    counts = np.zeros((Hkv,), np.int32)
    for r in range(Hkv):
        pages = [p for kb in t128[r, :c128[r]] for p in (2 * kb, 2 * kb + 1) if p < cap64]
        table[r, :len(pages)] = pages
        counts[r] = len(pages)
    assert (counts < cap64).any(), "the case should drop blocks"
    ref = oracle.attention(bits(q), bits(_pad_keys(k, cap64)), bits(_pad_keys(v, cap64)), [past // 64], table, counts,
                           SCALE)
    err = np.abs(f32(out) - ref)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())
    # the vendor functions at block 128
    mk = flash_prefill_compute_mean_k(k.to(gpu), block_size=128)
    assert float_bits_equal(f32(mk.permute(0, 2, 1, 3)), k128)
    scg = flash_prefill_score_chunked_from_mean_k(q.to(gpu), mk, key_len=kv_len, block_size=128)
    assert float_bits_equal(f32(scg.permute(0, 3, 1, 2)), sc)
    # a mean-K cache at block 128 gives the same output
    out2, _ = flashprefill_compactattn_prefill_full_kv(
        q.to(gpu), k.to(gpu), v.to(gpu), None, softmax_scale=SCALE, num_key_value_groups=G, block_size=128,
        pack_impl="indexed_dense", indexed_impl="fa2_paged", cache_fill_backend="auto", mean_k_cache=mk, **fp)
    assert torch.equal(out2, out)


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


GATE_CASES = [
    # (gate type, force_double, kv_group_aware_query)
    ("Qavg_Kavg", True, False),          # BASELINE config 1's gate
    ("Qavg_Kmaxminavg", False, False),   # the reference's default: no query projection, W_k per Q head
    ("Qavg_Kmaxminavg", True, False),
    ("Qmaxavg_Kmax", False, False),      # two query pools: projected per Q head
    ("Qavg_Kmaxminavg", False, True),    # kv-group-aware query, scores per KV head
]


@pytest.mark.parametrize("case", GATE_CASES, ids=lambda c: f"{c[0]}-fd{int(c[1])}-kv{int(c[2])}")
def test_attn_gate_bit_exact(gpu, case):
    """AttnGate scores for the reference's gate types against the oracle composition: pooling
    (max/min/avg, concatenated in that order), the reference's projection case for the type
    (attn_gate.py:74-86), block RoPE, q.k^T * 128^-1/2, causal softmax -- bit for bit."""
    gate_type, force_double, kv_aware = case
    _print_case(test="attn_gate", gate_type=gate_type, force_double=force_double, kv_aware=kv_aware)
    Hq, Hkv, Lq, past = 8, 2, 128, 64 * 12
    ch = make_chunk([past], Lq, Hq, Hkv, seed=8)
    gate = ATTNGATE_CLASSES[gate_type](64, 128, 128, Hkv, Hq, force_double=force_double,
                                       kv_group_aware_query=kv_aware).to(gpu)
    gate.reset_parameters(0.02, torch.Generator().manual_seed(2))
    cos, sin = rope_tables(ch.kv_cap)
    scores = gate(ch.q.to(gpu), _seq_first(ch.k).to(gpu), position_embeddings=(cos.to(gpu), sin.to(gpu)))
    P = ch.past_blocks
    assert gate.key_heads == (Hq if (gate_type == "Qavg_Kmaxminavg" and not force_double and not kv_aware) else Hkv)
    qg, kg = oracle_gate_summaries(gate, bits(ch.q), bits(_seq_first(ch.k)), f32(cos), f32(sin), P[0])
    assert tuple(scores.shape) == (1, gate.query_heads, Lq // 64, ch.kv_cap)
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


def test_paged_cache_summaries_after_decode_steps(gpu):
    """Decode appends complete a block without summaries; the next chunk append recomputes its
    mean-K from the cached keys, so every kmean equals a fresh computation over the whole
    sequence (a stale or zero summary would differ); gate-K cannot be recomputed (the cache
    has no pre-RoPE keys), so a gate append after such a block raises.  reset(keep_pages=True)
    starts the counts again and the next sequence's summaries are its own."""
    _print_case(test="paged_cache_summaries_after_decode")
    Hkv = 2
    g = torch.Generator().manual_seed(13)
    wk = (torch.randn((Hkv, 128, 128), generator=g) * 0.02).float().to(gpu)
    cos, sin = rope_tables(20)
    cos, sin = cos.to(gpu), sin.to(gpu)
    cache = PagedKVCache(1, Hkv, 64 * 12, gpu, with_kmean=True, with_kgate=True)
    for seq in range(2):
        parts = [torch.randn((1, n, Hkv, 128), generator=g).to(torch.bfloat16) for n in (320, 37, 27, 128)]
        cache.append(parts[0].to(gpu), parts[0].to(gpu), gate_wk=wk, rope_cos=cos, rope_sin=sin)
        cache.append_tokens(parts[1].to(gpu), parts[1].to(gpu))
        cache.append_tokens(parts[2].to(gpu), parts[2].to(gpu))
        assert (cache.length, cache.kmean_blocks, cache.kgate_blocks) == (384, 5, 5)
        with pytest.raises(ValueError, match="gate-K summaries are missing"):
            cache.append(parts[3].to(gpu), parts[3].to(gpu), gate_wk=wk, rope_cos=cos, rope_sin=sin)
        assert cache.length == 384
        cache.append(parts[3].to(gpu), parts[3].to(gpu))
        assert (cache.length, cache.kmean_blocks) == (512, 8)
        allk = torch.cat(parts, dim=1)
        assert torch.equal(cache.k_hf().cpu(), allk.transpose(1, 2))
        assert float_bits_equal(f32(cache.kmean[:, :, :8]), oracle.block_mean(bits(allk)))
        cache.reset(keep_pages=True)
        assert (cache.length, cache.kmean_blocks, cache.kgate_blocks) == (0, 0, 0)
