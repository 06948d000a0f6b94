"""compactattn operator entry points (SeerAttention selector side).

Mirrors the reference's public API in compact_attn/modules/attention_forward_chunked_dense.py:
  chunked_prefill_column_dense_attention_forward        (:2732-2912)
  chunked_prefill_column_dense_attention_from_keep_block (:2147-2729)
with the same argument names, meanings and ValueError behaviour.  The execution behind
them is one path: HIP selection (strict threshold on the gate scores over causal query
blocks, Q-block union, current chunk open), GQA union + ascending compaction into int32
block tables, and the HIP indexed MFMA attention reading K/V in place through the tables.
pack_impl / indexed_impl / cache_fill_backend are validated like the reference and then
all map to that path.

Selection (the reference's _build_keep_block_mask_chunked_fast_path + _build_kv_head_union_
keep_block_mask, :559-683): a past block is kept for a Q head when some query block's gate score
is strictly above the threshold, the last keep_recent_blocks KV blocks are forced (the current
chunk's blocks, then the past blocks right before it when keep_recent_blocks exceeds the
chunk's block count), the current chunk is always attended, and the KV group takes the union
of its Q heads.  The threshold is a float or a tensor with one value per request (:383-393).

Supported inputs (anything else raises ValueError): block_size 64, no padding in
attention_mask, head_dim 128, bf16 Q/K/V on the GPU.  A chunk whose length is not a multiple
of 64 selects and attends through the same path, its last block holding q_len % 64 tokens:
its queries see the selected past blocks and the current chunk causally, as the reference's
padded indexed path intends (_maybe_pad_indexed_dense_tail_inputs, :438-491; that path
aligns flash-attn's bottom-right causal mask to the padded key length, so each of its
queries also sees the next 64 - q_len % 64 positions, future tokens or zero-padded keys --
here the mask is at the true positions).  A chunk that starts inside a block (after decode
steps) attends densely when it has at most 64 queries, and raises otherwise.
"""
from __future__ import annotations

import os
from typing import Dict, List, Optional, Tuple, Union

import torch

from .. import ops
from ._core import (COMPACTATTN_VERSION, INDEXED_IMPLS, StageTimer, attend, check_attention_mask, dense_tables,
                    dense_tail, geometry, kv_layouts, starts_mid_block, table_stats)

PACK_IMPLS = frozenset({"torch", "triton", "indexed_dense"})
CACHE_FILL_BACKENDS = frozenset({"auto", "cuda", "triton"})


def _compactattn_effective_threshold(threshold: Union[float, torch.Tensor]) -> Union[float, torch.Tensor]:
    """A tensor passes through; a float can be replaced by the
    SEERATTN_DEBUG_COMPACTATTN_THRESHOLD_OVERRIDE environment value (reference :115-124)."""
    if isinstance(threshold, torch.Tensor):
        return threshold
    raw = os.environ.get("SEERATTN_DEBUG_COMPACTATTN_THRESHOLD_OVERRIDE")
    if raw is not None:
        try:
            return float(raw)
        except ValueError:
            pass
    return float(threshold)


def _compactattn_keep_recent_blocks(default: int) -> int:
    """keep_recent_blocks, or the SEERATTN_DEBUG_COMPACTATTN_KEEP_RECENT_OVERRIDE environment value
    (clamped at 0; reference :141-148)."""
    raw = os.environ.get("SEERATTN_DEBUG_COMPACTATTN_KEEP_RECENT_OVERRIDE")
    if raw is not None:
        try:
            return max(int(raw), 0)
        except ValueError:
            pass
    return int(default)


def keep_recent_local_blocks(keep_recent_blocks: int, q_blocks: int) -> int:
    """Forcing the last keep_recent_blocks of the P + Qb KV blocks (reference :632-636) keeps the
    Qb current blocks (always kept here) and, beyond them, the keep_recent_blocks - Qb past blocks
    right before the chunk: the selection rule's local_blocks."""
    return max(0, int(keep_recent_blocks) - int(q_blocks))


def request_thresholds(threshold: Union[float, torch.Tensor], batch: int) -> List[float]:
    """One threshold per request: a float or one-element tensor for all, or a 1-D tensor of
    ``batch`` values (the reference broadcasts view(-1, 1, 1) over [B, H, Kb], :383-393)."""
    if not isinstance(threshold, torch.Tensor):
        return [float(threshold)] * batch
    if threshold.dim() > 1:
        raise ValueError(f"Expected scalar or 1D batch threshold tensor, got shape={tuple(threshold.shape)}")
    vals = [float(x) for x in threshold.detach().float().cpu().reshape(-1).tolist()]
    if len(vals) == 1:
        return vals * batch
    if len(vals) != batch:
        raise ValueError(f"threshold tensor has {len(vals)} values for a batch of {batch}")
    return vals


def _full_width_scores(scores: torch.Tensor, kv_blocks: int) -> torch.Tensor:
    """Gate scores over fewer than kv_blocks key blocks cover the last columns (the reference
    right-aligns a short keep mask, _project_short_qhead_keep_block_to_kv_full_width,
    :708-734); the missing leading columns read as -inf, which no threshold keeps."""
    short = scores.shape[-1]
    if short >= kv_blocks:
        return scores
    full = torch.full((*scores.shape[:-1], kv_blocks), float("-inf"), dtype=scores.dtype, device=scores.device)
    full[..., kv_blocks - short:] = scores
    return full


def _validate_impls(pack_impl: str, indexed_impl: str, cache_fill_backend: str) -> None:
    if indexed_impl not in INDEXED_IMPLS:
        raise ValueError(f"Unsupported indexed_impl: {indexed_impl}")
    if pack_impl not in PACK_IMPLS:
        raise ValueError(f"Unsupported pack_impl: {pack_impl}")
    if cache_fill_backend not in CACHE_FILL_BACKENDS:
        raise ValueError(f"Unsupported cache_fill_backend: {cache_fill_backend}")


def _dense_mid_block(query_states, key_states, value_states, attention_mask, k_hf, v_hf, kv_len: int,
                     num_kv_heads: int, softmax_scale, return_stats: bool):
    """A chunk of at most 64 queries that starts inside a block attends densely to all kv_len
    keys (dense_tail); no selection can align its query block with the key blocks."""
    check_attention_mask(attention_mask, query_states.shape[0], kv_len)
    K, V = kv_layouts(key_states, value_states, k_hf, v_hf)
    out = dense_tail(query_states, K, V, kv_len, num_kv_heads, softmax_scale)
    if not return_stats:
        return out, None
    return out, {"compactattn_version": COMPACTATTN_VERSION, "col_dense_tail_tokens": float(query_states.shape[1])}


def chunked_prefill_column_dense_attention_forward(
    query_states: torch.Tensor,  # [B, Q, Hq, D]
    key_states: torch.Tensor,  # [B, K, Hkv, D]
    value_states: torch.Tensor,  # [B, K, Hkv, D]
    attention_mask: Optional[torch.Tensor],  # [B, K]
    query_length: int,
    softmax_scale: Optional[float] = None,
    attn_gate_score: Optional[torch.Tensor] = None,  # [B, Hq|Hkv, Qb, Kb]
    block_attention_mask: Optional[torch.Tensor] = None,  # [B, 1, Qb, Kb]
    threshold: Union[float, torch.Tensor] = 0.0,
    keep_recent_blocks: int = 2,
    block_size: int = 64,
    num_key_value_groups: int = 1,
    attn_gate_is_kv_group_aware: bool = False,
    pack_impl: str = "torch",
    indexed_impl: str = "fa2_paged",
    cache_fill_backend: str = "auto",
    return_stats: bool = False,
    attn_module=None,
    k_hf: Optional[torch.Tensor] = None,  # [B, Hkv, K, D] heads-first
    v_hf: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[Dict[str, float]]]:
    """Seer compactattn: keep KV block kb for Q head h iff max over the causal query blocks
    of attn_gate_score[b, h, qb, kb] > threshold (reference: _build_keep_block_mask /
    build_keep_past_fast, attention_forward_chunked_dense.py:352-403,559-638), force the
    last keep_recent_blocks KV blocks and the current chunk open, union over the GQA group,
    then attend over the selected blocks.

    block_attention_mask, when given, must be the standard causal block mask (the path
    applies causality itself).  A threshold tensor holds one value per request; with it the
    past columns' validity is the causal block mask here too (the reference's generic path
    takes a top-left triangle when block_attention_mask is None)."""
    del attn_module, block_attention_mask
    if attn_gate_score is None:
        raise ValueError("attn_gate_score is required for chunked column-dense attention.")
    if query_length <= 1:
        raise ValueError("chunked_prefill_column_dense_attention_forward expects query_length > 1.")
    if block_size <= 0:
        raise ValueError("block_size must be positive.")
    _validate_impls(pack_impl, indexed_impl, cache_fill_backend)
    threshold = _compactattn_effective_threshold(threshold)
    keep_recent_blocks = _compactattn_keep_recent_blocks(keep_recent_blocks)
    kv_len = k_hf.shape[2] if k_hf is not None else key_states.shape[1]
    num_kv_heads = k_hf.shape[1] if k_hf is not None else key_states.shape[2]
    if query_states.dim() == 4 and query_states.shape[1] != query_length:
        raise ValueError(f"query_length={query_length} does not match query_states ({query_states.shape[1]})")
    if block_size == 64 and starts_mid_block(query_states.shape[1], kv_len):
        return _dense_mid_block(query_states, key_states, value_states, attention_mask, k_hf, v_hf, kv_len,
                                num_kv_heads, softmax_scale, return_stats)
    geo = geometry(query_states, kv_len, num_kv_heads, block_size)
    if geo.q_len != query_length:
        raise ValueError(f"query_length={query_length} does not match query_states ({geo.q_len})")
    if geo.group != num_key_value_groups:
        raise ValueError(f"num_key_value_groups={num_key_value_groups} does not match heads "
                         f"{geo.num_q_heads}/{geo.num_kv_heads}")
    check_attention_mask(attention_mask, geo.batch, kv_len)
    if keep_recent_blocks < 0:
        raise ValueError("keep_recent_blocks must be >= 0")
    thresholds = request_thresholds(threshold, geo.batch)
    K, V = kv_layouts(key_states, value_states, k_hf, v_hf)
    timer = StageTimer(return_stats)
    P = [geo.past_blocks] * geo.batch

    if geo.past_blocks == 0:  # first chunk: dense causal (reference: kv_len == q_len path)
        table, counts = dense_tables(geo, query_states.device)
    else:
        sel_heads = geo.num_kv_heads if attn_gate_is_kv_group_aware else geo.num_q_heads
        if attn_gate_score.dim() != 4 or attn_gate_score.shape[0] != geo.batch or \
                attn_gate_score.shape[1] != sel_heads or attn_gate_score.shape[2] != geo.q_blocks:
            raise ValueError(f"attn_gate_score must be [B, {sel_heads}, {geo.q_blocks}, Kb], got "
                             f"{tuple(attn_gate_score.shape)}")
        short = attn_gate_score.shape[3]
        if short > geo.kv_cap:
            raise ValueError(f"short keep_block width {short} exceeds expected KV blocks {geo.kv_cap}")
        scores = attn_gate_score if attn_gate_score.stride(-1) == 1 else attn_gate_score.contiguous()
        if scores.dtype not in (torch.float32, torch.bfloat16):
            scores = scores.float()
        scores = _full_width_scores(scores, geo.kv_cap)
        # the forced recent columns of a short score row stop at its first column
        local = keep_recent_local_blocks(min(keep_recent_blocks, short), geo.q_blocks)

        def select():
            # kv-group-aware gates score per KV head: selection then runs with G = 1
            if len(set(thresholds)) == 1:
                return ops.select_scores(scores, ops.Rule(threshold=thresholds[0], local_blocks=local), P,
                                         geo.num_kv_heads, geo.kv_cap, geo.q_len)
            return torch.cat([ops.select_scores(scores[b:b + 1], ops.Rule(threshold=t, local_blocks=local), P[b:b + 1],
                                                geo.num_kv_heads, geo.kv_cap, geo.q_len)
                              for b, t in enumerate(thresholds)])

        rowmask = timer("col_select_mask_ms", select)
        table, counts, _, _ = timer("col_union_table_ms", lambda: ops.union_compact(
            rowmask, P, geo.num_kv_heads, geo.kv_cap))
    out = timer("col_index_attn_ms", lambda: attend(query_states, K, V, table, counts, geo, softmax_scale))
    if not return_stats:
        return out, None
    thr_stat = float(threshold) if not isinstance(threshold, torch.Tensor) else float(threshold.float().mean())
    stats: Dict[str, float] = {"compactattn_version": COMPACTATTN_VERSION, "col_threshold": thr_stat}
    stats.update(timer.results())
    stats.update(table_stats(counts, geo, "col_"))
    return out, stats


def chunked_prefill_column_dense_attention_from_keep_block(
    query_states: torch.Tensor,  # [B, Q, Hq, D]
    key_states: torch.Tensor,  # [B, K, Hkv, D]
    value_states: torch.Tensor,  # [B, K, Hkv, D]
    keep_block: Optional[torch.Tensor],  # [B, Hq, Kb]
    attention_mask: Optional[torch.Tensor],  # [B, K]
    query_length: int,
    softmax_scale: float,
    block_size: int = 64,
    num_key_value_groups: int = 1,
    pack_impl: str = "torch",
    indexed_impl: str = "fa2_paged",
    cache_fill_backend: str = "auto",
    return_stats: bool = False,
    valid_block: Optional[torch.Tensor] = None,  # [B, Hq, Kb]
    allow_indexed_dense: bool = False,
    keep_block_kv_preprojected: Optional[torch.Tensor] = None,  # [B, Hkv, Kb]
    attn_module=None,
    k_hf: Optional[torch.Tensor] = None,
    v_hf: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[Dict[str, float]]]:
    """Attention over caller-selected blocks: keep_block (per Q head, OR-ed over the GQA
    group and AND-ed with valid_block) or keep_block_kv_preprojected (per KV group).  The
    current chunk is always attended (causally)."""
    del attn_module, allow_indexed_dense
    if query_length <= 1:
        raise ValueError("chunked_prefill_column_dense_attention_from_keep_block expects query_length > 1.")
    if block_size <= 0:
        raise ValueError("block_size must be positive.")
    _validate_impls(pack_impl, indexed_impl, cache_fill_backend)
    kv_len = k_hf.shape[2] if k_hf is not None else key_states.shape[1]
    num_kv_heads = k_hf.shape[1] if k_hf is not None else key_states.shape[2]
    if query_states.dim() == 4 and query_states.shape[1] != query_length:
        raise ValueError(f"query_length={query_length} does not match query_states ({query_states.shape[1]})")
    if block_size == 64 and starts_mid_block(query_states.shape[1], kv_len):
        return _dense_mid_block(query_states, key_states, value_states, attention_mask, k_hf, v_hf, kv_len,
                                num_kv_heads, softmax_scale, return_stats)
    geo = geometry(query_states, kv_len, num_kv_heads, block_size)
    if geo.q_len != query_length:
        raise ValueError(f"query_length={query_length} does not match query_states ({geo.q_len})")
    if geo.group != num_key_value_groups:
        raise ValueError(f"num_key_value_groups={num_key_value_groups} does not match heads "
                         f"{geo.num_q_heads}/{geo.num_kv_heads}")
    if keep_block is None and keep_block_kv_preprojected is None:
        raise ValueError("Either keep_block or keep_block_kv_preprojected must be provided.")
    kv_blocks = geo.kv_cap
    if keep_block is not None and tuple(keep_block.shape) != (geo.batch, geo.num_q_heads, kv_blocks):
        raise ValueError(f"keep_block shape mismatch: expected {(geo.batch, geo.num_q_heads, kv_blocks)}, "
                         f"got {tuple(keep_block.shape)}")
    if keep_block_kv_preprojected is not None and \
            tuple(keep_block_kv_preprojected.shape) != (geo.batch, geo.num_kv_heads, kv_blocks):
        raise ValueError(f"keep_block_kv_preprojected shape mismatch: expected "
                         f"{(geo.batch, geo.num_kv_heads, kv_blocks)}, got {tuple(keep_block_kv_preprojected.shape)}")
    check_attention_mask(attention_mask, geo.batch, kv_len)
    K, V = kv_layouts(key_states, value_states, k_hf, v_hf)
    timer = StageTimer(return_stats)
    P = [geo.past_blocks] * geo.batch

    def keep_kv_mask() -> torch.Tensor:
        if keep_block_kv_preprojected is not None:
            return keep_block_kv_preprojected.to(torch.bool).contiguous()
        kb = keep_block.to(torch.bool)
        if valid_block is not None:
            kb = kb & valid_block.to(torch.bool)
        return kb.view(geo.batch, geo.num_kv_heads, geo.group, kv_blocks).any(dim=2).contiguous()

    keep_kv = timer("col_gqa_union_ms", keep_kv_mask)
    table, counts = timer("col_union_table_ms", lambda: ops.compact_keep_kv(
        keep_kv, P, geo.q_len, geo.num_q_heads, geo.kv_cap))
    out = timer("col_index_attn_ms", lambda: attend(query_states, K, V, table, counts, geo, softmax_scale))
    if not return_stats:
        return out, None
    stats: Dict[str, float] = {"compactattn_version": COMPACTATTN_VERSION}
    stats.update(timer.results())
    stats.update(table_stats(counts, geo, "col_"))
    return out, stats
