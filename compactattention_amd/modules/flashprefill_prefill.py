"""FlashPrefill compactattn entry point.

Mirrors flashprefill_compactattn_prefill_full_kv of the reference
(compact_attn/modules/flashprefill_prefill.py:880-1189) -- same keyword arguments and
return value -- with the selection of _flashprefill_keep_block_from_scores_rowwise
(:596-666): per (Q head, query block) row, keep score >= alpha * rowmax, the sink blocks
(kb < attention_sink), the window (0 <= q_abs - kb < window_size) and, with min_budget > 0,
the top-min_budget columns of the row by (score desc, block id asc), ranked over all Kb key
blocks with non-causal and non-finite entries read as 0 (torch.topk over the zeroed row,
:633-647; picks past the causal edge are dropped); rows of the last
last_n_block query blocks stay out of the union; the current chunk is always kept; then
the GQA union, int32 block tables and the indexed attention.

Score blocks are 64 or 128 tokens (block_size; 128 is the reference's default).  Pages,
tables and attention stay in 64-token blocks: 128-token scoring pools pairs of 64-token
summaries (ca_pair_block_summaries), applies the rule in 128-token block units (sink, window,
min_budget and last_n_block count 128-token blocks, as in the reference) and names both
64-token pages of every selected 128-token block.  A 128-token chunk must start at a multiple
of 128 tokens.

Scores are the pooled softmax of flash_prefill_score_chunked_from_mean_k (see
compactattention_amd.flashprefill_vendor) by default; score_mode="token" (a keyword of this
build) scores the chunk's query tokens against the key means as the reference's
compute_block_score_chunked + normalize_scores do (flashprefill_native_forward.py:98-207,
365-374), on bf16 MFMAs.  A first chunk (kv_len == q_len) runs dense causal
attention on the same HIP kernel (identity tables); q_len <= 1 attends densely through the
decode kernel, where the reference calls its dense backend (q_len <= 1 or kv_len <= q_len,
:903-907).  A chunk whose length is not a multiple of the block size selects and attends with
a partial last block (its summaries pool its valid tokens); one that starts inside a 64-token
block (after decode steps) attends densely (at most 64 queries).
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Sequence, Tuple

import torch

from .. import ops
from ..flashprefill_vendor import mean_k_kernel_layout
from ._core import (COMPACTATTN_VERSION, INDEXED_IMPLS, StageTimer, attend, check_attention_mask, dense_tables,
                    dense_tail, geometry, kv_layouts, starts_mid_block, table_stats)
from .attention_forward_chunked_dense import CACHE_FILL_BACKENDS, PACK_IMPLS

SCORE_BLOCK_SIZES = (64, 128)


def flashprefill_rule(attention_sink: int, window_size: int, alpha: float, last_n_block: int,
                      min_budget: int) -> ops.Rule:
    return ops.Rule(topk=max(int(min_budget), 0), alpha=float(alpha), sink_blocks=int(attention_sink),
                    window_blocks=int(window_size), last_n_block=int(last_n_block), topk_all_columns=True)


def check_score_block_size(block_size: int) -> None:
    if block_size not in SCORE_BLOCK_SIZES:
        raise ValueError(f"block_size={block_size}: FlashPrefill scoring runs 64- or 128-token blocks")


def expand_pair_tables(table: torch.Tensor, counts: torch.Tensor, key_blocks: int, kv_cap: int
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Tables of 128-token blocks -> tables of 64-token pages: block k names pages 2k and 2k + 1,
    in order; when key_blocks (the 64-token blocks of each row) is odd, the last 128-token block
    (the current chunk's, closing every row) has page 2k only.  Entries past the counts are -1."""
    rows = table.shape[0]
    t = table.to(torch.int64)
    pages = torch.stack([2 * t, 2 * t + 1], dim=-1).reshape(rows, -1)
    cnt = 2 * counts.to(torch.int64) - (key_blocks % 2)
    out = torch.full((rows, kv_cap), -1, dtype=torch.int32, device=table.device)
    width = min(kv_cap, pages.shape[1])
    keep = torch.arange(width, device=table.device)[None, :] < cnt[:, None]
    out[:, :width] = torch.where(keep, pages[:, :width], torch.full_like(pages[:, :width], -1)).to(torch.int32)
    return out, cnt.to(torch.int32)


SCORE_MODES = ("pooled", "token")


def check_score_mode(score_mode: str) -> None:
    if score_mode not in SCORE_MODES:
        raise ValueError(f"score_mode={score_mode!r}: expected one of {SCORE_MODES}")


def token_mass_rowmask(query_states: torch.Tensor, khat: torch.Tensor, past: Sequence[int], num_kv_heads: int,
                       cap: int, rule: ops.Rule, block_size: int) -> torch.Tensor:
    """Row masks from the reference's per-token scores (ca_score_token_mass) in block_size blocks:
    past and cap count block_size blocks, khat holds block_size-token key means."""
    scale = 1.0 / math.sqrt(128)
    scores = ops.score_token_mass(query_states, khat.contiguous(), scale, past, num_kv_heads, cap, block_size)
    return ops.select_scores(scores, rule, past, num_kv_heads, cap, 64 * scores.shape[2])


def flashprefill_tables(qhat: torch.Tensor, khat: torch.Tensor, past_blocks: Sequence[int], q_len: int,
                        num_kv_heads: int, kv_cap: int, rule: ops.Rule, block_size: int,
                        khat_block_size: int = 64, score_mode: str = "pooled",
                        query_states: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-KV-group tables of 64-token page ids for a chunk of q_len tokens at past_blocks
    (64-token blocks, one value for every request).  qhat [B, Hq, ceil(q_len/64), 128] are the
    chunk's 64-token query means; khat [B, Hkv, >= P + Qb, 128] the key means in
    khat_block_size-token blocks (a 128-token khat goes straight to the 128-token scoring).
    score_mode "pooled" scores the block means (the bit-reproducible form); "token" scores the
    chunk's query tokens against the key means as the reference does (query_states
    [B, q_len, Hq, 128] required, qhat unused)."""
    check_score_block_size(block_size)
    check_score_mode(score_mode)
    if score_mode == "token" and query_states is None:
        raise ValueError("score_mode='token' needs query_states")
    scale = 1.0 / math.sqrt(128)
    P = [int(p) for p in past_blocks]
    if block_size == 64:
        if score_mode == "token":
            rowmask = token_mass_rowmask(query_states, khat[..., :kv_cap, :], P, num_kv_heads, kv_cap, rule, 64)
        else:
            rowmask, _ = ops.score_select(qhat, khat, scale, rule, P, num_kv_heads, kv_cap)
        table, counts, _, _ = ops.union_compact(rowmask, P, num_kv_heads, kv_cap, last_n_block=rule.last_n_block)
        return table, counts
    if len(set(P)) != 1 or P[0] % 2:
        raise ValueError(f"128-token FlashPrefill blocks need a chunk that starts at a multiple of 128 tokens "
                         f"(past {64 * P[0]} tokens)")
    qb64 = -(-q_len // 64)
    last = q_len - 64 * (qb64 - 1)  # tokens of the chunk's last 64-token block
    kb64 = P[0] + qb64
    q128 = ops.pair_block_summaries(qhat, qb64, last) if score_mode == "pooled" else None
    P128 = [P[0] // 2] * len(P)
    cap128 = -(-kb64 // 2)
    if khat_block_size == 128:  # rows of exactly cap128 summaries (the kernels' row stride)
        k128 = khat[..., :cap128, :].contiguous()
    else:
        k128 = ops.pair_block_summaries(khat, kb64, last)
    if score_mode == "token":
        rowmask = token_mass_rowmask(query_states, k128, P128, num_kv_heads, cap128, rule, 128)
    else:
        rowmask, _ = ops.score_select(q128, k128, scale, rule, P128, num_kv_heads, cap128)
    t128, c128, _, _ = ops.union_compact(rowmask, P128, num_kv_heads, cap128, last_n_block=rule.last_n_block)
    return expand_pair_tables(t128, c128, kb64, kv_cap)


def flashprefill_compactattn_prefill_full_kv(
    query_states: torch.Tensor,
    key_states: torch.Tensor,
    value_states: torch.Tensor,
    attention_mask: Optional[torch.Tensor],
    *,
    softmax_scale: float,
    num_key_value_groups: int,
    block_size: int,
    attention_sink: int,
    window_size: int,
    alpha: float,
    last_n_block: int,
    min_budget: int,
    pack_impl: str,
    indexed_impl: str,
    cache_fill_backend: str,
    measure_timing: bool = False,
    attn_module=None,
    k_hf: Optional[torch.Tensor] = None,
    v_hf: Optional[torch.Tensor] = None,
    mean_k_cache: Optional[torch.Tensor] = None,
    score_mode: str = "pooled",
) -> Tuple[torch.Tensor, Dict[str, float]]:
    del attn_module
    check_score_mode(score_mode)
    if indexed_impl not in INDEXED_IMPLS:
        raise ValueError(f"Unsupported indexed_impl: {indexed_impl}")
    if pack_impl not in PACK_IMPLS:
        raise ValueError(f"Unsupported pack_impl: {pack_impl}")
    if cache_fill_backend not in CACHE_FILL_BACKENDS:
        raise ValueError(f"Unsupported cache_fill_backend: {cache_fill_backend}")
    check_score_block_size(block_size)
    kv_len = k_hf.shape[2] if k_hf is not None else key_states.shape[1]
    num_kv_heads = k_hf.shape[1] if k_hf is not None else key_states.shape[2]
    q_len = query_states.shape[1]
    if q_len <= 1 or starts_mid_block(q_len, kv_len):
        # the reference's dense fallback for q_len <= 1 (:903-907); a chunk starting inside a block
        check_attention_mask(attention_mask, query_states.shape[0], kv_len)
        K, V = kv_layouts(key_states, value_states, k_hf, v_hf)
        out = dense_tail(query_states, K, V, kv_len, num_kv_heads, softmax_scale)
        return out, {"compactattn_version": COMPACTATTN_VERSION, "flashprefill_dense_calls": 1.0,
                     "flashprefill_dense_tail_tokens": float(q_len)}
    geo = geometry(query_states, kv_len, num_kv_heads, 64)
    if geo.group != num_key_value_groups:
        raise ValueError(f"num_key_value_groups={num_key_value_groups} does not match heads "
                         f"{geo.num_q_heads}/{geo.num_kv_heads}")
    check_attention_mask(attention_mask, geo.batch, kv_len)
    K, V = kv_layouts(key_states, value_states, k_hf, v_hf)
    timer = StageTimer(measure_timing)
    P = [geo.past_blocks] * geo.batch
    stats: Dict[str, float] = {"compactattn_version": COMPACTATTN_VERSION}

    if geo.past_blocks == 0:
        table, counts = dense_tables(geo, query_states.device)
        out = timer("attention_ms", lambda: attend(query_states, K, V, table, counts, geo, softmax_scale))
        stats["flashprefill_dense_calls"] = 1.0
        stats.update(timer.results())
        return out, stats
    if block_size == 128 and geo.past_blocks % 2:
        raise ValueError(f"128-token FlashPrefill blocks need a chunk that starts at a multiple of 128 tokens "
                         f"(past {kv_len - q_len} tokens)")

    def summaries():
        """Key means in 64-token blocks, or the caller's mean_k_cache in block_size blocks."""
        if mean_k_cache is not None:
            m = mean_k_kernel_layout(mean_k_cache)
            need = -(-kv_len // block_size)
            if m.shape[2] < need:
                raise ValueError(f"mean_k_cache covers {m.shape[2]} blocks, need {need}")
            return m, block_size
        # no cache: block means of the whole key range (what the reference recomputes too)
        m = torch.empty((geo.batch, geo.num_kv_heads, geo.kv_cap, 128), dtype=torch.float32,
                        device=query_states.device)
        ks = key_states if key_states is not None else k_hf.transpose(1, 2)
        ops.cache_fill(ks, None, None, None, [0] * geo.batch, geo.kv_cap, m)
        return m, 64

    khat, khat_bs = timer("mean_k_ms", summaries)
    rule = flashprefill_rule(attention_sink, window_size, alpha, last_n_block, min_budget)

    def select():
        cap = khat.shape[2] if khat_bs == 64 else geo.kv_cap
        qhat = ops.pool_query(query_states, P, cap, num_kv_heads=geo.num_kv_heads)
        return flashprefill_tables(qhat, khat, P, geo.q_len, geo.num_kv_heads, cap, rule, block_size,
                                   khat_block_size=khat_bs, score_mode=score_mode, query_states=query_states)

    table, counts = timer("flashprefill_select_ms", select)
    out = timer("attention_ms", lambda: attend(query_states, K, V, table, counts, geo, softmax_scale))
    if measure_timing:
        stats.update(timer.results())
        stats.update(table_stats(counts, geo, "flashprefill_"))
    return out, stats
