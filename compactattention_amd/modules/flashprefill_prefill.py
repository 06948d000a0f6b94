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

Scores are the pooled softmax of flash_prefill_score_chunked_from_mean_k (see
compactattention_amd.flashprefill_vendor).  A first chunk (kv_len == q_len) runs dense causal
attention on the same HIP kernel (identity tables), and a call with fewer than 64 queries
attends densely through the decode kernel, where the reference calls its dense backend
(q_len <= 1 or kv_len <= q_len, :903-907).  A longer chunk whose length is not a multiple of
64 selects for its block-aligned head and runs its last q_len % 64 queries densely.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from .. import ops
from ..flashprefill_vendor import mean_k_kernel_layout
from ._core import (COMPACTATTN_VERSION, INDEXED_IMPLS, StageTimer, aligned_head, attend, check_attention_mask,
                    dense_tables, dense_tail, geometry, kv_layouts, table_stats)
from .attention_forward_chunked_dense import CACHE_FILL_BACKENDS, PACK_IMPLS


def flashprefill_rule(attention_sink: int, window_size: int, alpha: float, last_n_block: int,
                      min_budget: int) -> ops.Rule:
    return ops.Rule(topk=max(int(min_budget), 0), alpha=float(alpha), sink_blocks=int(attention_sink),
                    window_blocks=int(window_size), last_n_block=int(last_n_block), topk_all_columns=True)


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
) -> Tuple[torch.Tensor, Dict[str, float]]:
    del attn_module
    if indexed_impl not in INDEXED_IMPLS:
        raise ValueError(f"Unsupported indexed_impl: {indexed_impl}")
    if pack_impl not in PACK_IMPLS:
        raise ValueError(f"Unsupported pack_impl: {pack_impl}")
    if cache_fill_backend not in CACHE_FILL_BACKENDS:
        raise ValueError(f"Unsupported cache_fill_backend: {cache_fill_backend}")
    kv_len = k_hf.shape[2] if k_hf is not None else key_states.shape[1]
    num_kv_heads = k_hf.shape[1] if k_hf is not None else key_states.shape[2]
    head = aligned_head(query_states.shape[1], kv_len) if block_size == 64 else None
    if head is not None:
        # fewer than 64 queries: dense over the whole KV (the reference's dense fallback for
        # q_len <= 1, :903-907); otherwise the aligned head selects and the tail is dense
        check_attention_mask(attention_mask, query_states.shape[0], kv_len)
        K, V = kv_layouts(key_states, value_states, k_hf, v_hf)
        stats: Dict[str, float] = {"compactattn_version": COMPACTATTN_VERSION}
        parts = []
        if head > 0:
            keep = kv_len - (query_states.shape[1] - head)
            cut = lambda t, dim: None if t is None else t.narrow(dim, 0, keep)  # noqa: E731
            out_head, stats = flashprefill_compactattn_prefill_full_kv(
                query_states[:, :head], cut(key_states, 1), cut(value_states, 1), cut(attention_mask, 1),
                softmax_scale=softmax_scale, num_key_value_groups=num_key_value_groups, block_size=block_size,
                attention_sink=attention_sink, window_size=window_size, alpha=alpha, last_n_block=last_n_block,
                min_budget=min_budget, pack_impl=pack_impl, indexed_impl=indexed_impl,
                cache_fill_backend=cache_fill_backend, measure_timing=measure_timing, k_hf=cut(k_hf, 2),
                v_hf=cut(v_hf, 2), mean_k_cache=mean_k_cache)
            parts.append(out_head)
        parts.append(dense_tail(query_states[:, head:], K, V, kv_len, num_kv_heads, softmax_scale))
        stats["flashprefill_dense_tail_tokens"] = float(query_states.shape[1] - head)
        return torch.cat(parts, dim=1) if len(parts) > 1 else parts[0], stats
    geo = geometry(query_states, kv_len, num_kv_heads, block_size)
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

    def summaries():
        if mean_k_cache is not None:
            m = mean_k_kernel_layout(mean_k_cache)
            if m.shape[2] < geo.kv_cap:
                raise ValueError(f"mean_k_cache covers {m.shape[2]} blocks, need {geo.kv_cap}")
            return m
        # no cache: block means of the whole key range (what the reference recomputes too)
        m = torch.empty((geo.batch, geo.num_kv_heads, geo.kv_cap, 128), dtype=torch.float32,
                        device=query_states.device)
        ks = key_states if key_states is not None else k_hf.transpose(1, 2)
        ops.cache_fill(ks, None, None, None, [0] * geo.batch, geo.kv_cap, m)
        return m

    khat = timer("mean_k_ms", summaries)
    rule = flashprefill_rule(attention_sink, window_size, alpha, last_n_block, min_budget)

    def select():
        qhat = ops.pool_query(query_states, P, khat.shape[2], num_kv_heads=geo.num_kv_heads)
        rowmask, _ = ops.score_select(qhat, khat, 1.0 / math.sqrt(128), rule, P, geo.num_kv_heads,
                                      khat.shape[2])
        return rowmask

    rowmask = timer("flashprefill_select_ms", select)
    table, counts, _, _ = timer("flashprefill_union_ms", lambda: ops.union_compact(
        rowmask, P, geo.num_kv_heads, khat.shape[2], last_n_block=last_n_block))
    out = timer("attention_ms", lambda: attend(query_states, K, V, table, counts, geo, softmax_scale))
    if measure_timing:
        stats.update(timer.results())
        stats.update(table_stats(counts, geo, "flashprefill_"))
    return out, stats
