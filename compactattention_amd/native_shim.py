"""Drop-in replacement for the reference's native-extension wrapper module.

Every `_C_compactattn` call of the reference goes through
compact_attn/kernels/varlen/indexed_dense_cache_fill_cuda.py: a `can_use_cuda_*` guard per
function (False sends the caller to its torch/Triton path) and a `*_cuda` wrapper around the
extension.  A maintainer who points the reference's own Python at this library installs this
module under that name.  Names and keyword arguments are kept:

  - the selection-side functions run on this library (ca_select_scores, ca_union_compact,
    ca_compact_keep_kv, ca_table_to_csr);
  - the gather side (selected-KV gathers, Q packing, gather-workspace page tables) has no
    counterpart, because ca_attn_fwd reads the selected pages of the cache in place: its
    guards return False and its wrappers raise.  The caller's indexed attention call is
    replaced by ca_attn_fwd as well (ops.attn_fwd), which makes those workspaces unnecessary.

Reference kernels restated here (compact_attn/csrc/compactattn/cache_fill_kernel.cu):
build_keep_past_fast :275-298, build_keep_curr_fast :301-326,
build_selected_indices_from_kv_keep_block :449-483, build_flashinfer_kv_indices :485-505.
"""
from __future__ import annotations

import torch

from . import _hip, ops

BLOCK = 64


def cuda_cache_fill_available() -> bool:
    try:
        _hip.lib()
        return True
    except (RuntimeError, OSError):
        return False


def can_use_cuda_keep_block_fast(attn_gate_score: torch.Tensor) -> bool:
    s = attn_gate_score
    return (cuda_cache_fill_available() and s.is_cuda and s.is_contiguous() and s.dim() == 4
            and s.dtype in (torch.float32, torch.bfloat16))


def can_use_cuda_build_selected_indices_from_kv_keep_block(keep_block_kv: torch.Tensor, *args, **kwargs) -> bool:
    return (cuda_cache_fill_available() and keep_block_kv.is_cuda and keep_block_kv.dim() == 3
            and keep_block_kv.dtype == torch.bool)


def can_use_cuda_build_flashinfer_kv_indices(selected_block_indices: torch.Tensor, *args, **kwargs) -> bool:
    return (cuda_cache_fill_available() and selected_block_indices.is_cuda
            and selected_block_indices.dtype == torch.int32)


def _no_counterpart(*args, **kwargs) -> bool:
    """Gathers, Q packing and gather-workspace page tables: the in-place attention replaces them."""
    return False


can_use_cuda_build_block_table = _no_counterpart
can_use_cuda_compact_keep_blocks = _no_counterpart
can_use_cuda_compact_keep_blocks_and_build_table = _no_counterpart
can_use_cuda_pack_q_for_indexed_prefill = _no_counterpart
can_use_cuda_cache_fill_from_pos_with_rank = _no_counterpart
can_use_cuda_cache_fill_from_pos_with_local_rank = _no_counterpart
can_use_cuda_cache_fill_from_row_blk_dst = _no_counterpart
can_use_cuda_cache_fill_from_selected_indices_row_tiled = _no_counterpart
can_use_cuda_keep_block_builder_fast = _no_counterpart


def _row_masks(attn_gate_score: torch.Tensor, threshold: float, past_k_blocks: int) -> torch.Tensor:
    """Threshold row masks [B, H, Qb, words] int32: bit kb of row (b, h, q) is score > threshold
    for the causal columns kb <= past_k_blocks + q."""
    if not can_use_cuda_keep_block_fast(attn_gate_score):
        raise ValueError("attn_gate_score must be a contiguous fp32/bf16 [B, H, Qb, Kb] GPU tensor")
    B, H, Qb, Kb = attn_gate_score.shape
    if Kb != past_k_blocks + Qb:
        raise ValueError(f"attn_gate_score has {Kb} key blocks, expected past {past_k_blocks} + {Qb} current")
    rule = ops.Rule(threshold=float(threshold))
    return ops.select_scores(attn_gate_score, rule, [int(past_k_blocks)] * B, H, Kb, Qb * BLOCK)


def build_keep_past_fast_cuda(*, attn_gate_score: torch.Tensor, threshold: float, past_k_blocks: int
                              ) -> torch.Tensor:
    """[B, H, P] bool: any query block's score above the threshold, per past column."""
    B, H, _, Kb = attn_gate_score.shape
    rowmask = _row_masks(attn_gate_score, threshold, past_k_blocks)
    _, _, keep_block, _ = ops.union_compact(rowmask, [int(past_k_blocks)] * B, H, Kb, want_keep_block=True)
    return keep_block[:, :, :past_k_blocks].bool()


def build_keep_curr_fast_cuda(*, attn_gate_score: torch.Tensor, threshold: float, past_k_blocks: int,
                              curr_k_blocks: int) -> torch.Tensor:
    """[B, H, C] bool: any causal query block's score above the threshold, per current column
    (a row mask holds no column past its causal edge, so the OR over all query blocks is the
    reference's OR over q >= c)."""
    rowmask = _row_masks(attn_gate_score, threshold, past_k_blocks)
    cols = torch.arange(past_k_blocks, past_k_blocks + curr_k_blocks, device=rowmask.device)
    bits = (rowmask[:, :, :, cols // 32] >> (cols % 32)) & 1  # [B, H, Qb, C]
    return bits.any(dim=2)


def build_selected_indices_from_kv_keep_block_cuda_out(*, keep_block_kv: torch.Tensor,
                                                       selected_block_indices: torch.Tensor,
                                                       selected_block_counts: torch.Tensor) -> None:
    """Ascending kept block ids per (b, kv head) row and their counts.  ca_compact_keep_kv
    always keeps a request's current blocks; with no chunk length in this signature the last
    column stands in as the one current block, and rows that did not keep it drop it again."""
    if not can_use_cuda_build_selected_indices_from_kv_keep_block(keep_block_kv):
        raise ValueError("keep_block_kv must be a bool [B, Hkv, Kb] GPU tensor")
    B, Hkv, Kb = keep_block_kv.shape
    keep = keep_block_kv.contiguous()
    table, counts = ops.compact_keep_kv(keep, [Kb - 1] * B, BLOCK, Hkv, Kb)
    drop = ~keep[:, :, Kb - 1].reshape(-1)
    counts = counts - drop.to(torch.int32)
    slot = counts.to(torch.int64).clamp(0, Kb - 1)[:, None]
    table.scatter_(1, slot, torch.where(drop[:, None], torch.full_like(slot, -1, dtype=torch.int32),
                                        table.gather(1, slot)))
    selected_block_indices[:, :Kb].copy_(table)
    selected_block_counts.copy_(counts)


def build_flashinfer_kv_indices_cuda_out(*, selected_block_indices: torch.Tensor,
                                         selected_block_counts: torch.Tensor, kv_indptr: torch.Tensor,
                                         kv_indices: torch.Tensor, kv_blocks: int) -> None:
    """kv_indices[kv_indptr[r] + i] = r * kv_blocks + selected_block_indices[r][i].  kv_indptr
    is the caller's exclusive prefix sum of the counts (as the reference's callers build it);
    ca_table_to_csr computes the same prefix sum on the device, and only kv_indices is written."""
    rows = selected_block_counts.shape[0]
    table = selected_block_indices[:, :kv_blocks]
    if table.shape[1] < kv_blocks:  # the kernel may read a row's first kv_blocks entries
        padded = torch.zeros((rows, kv_blocks), dtype=table.dtype, device=table.device)
        padded[:, :table.shape[1]] = table
        table = padded
    elif table.stride(1) != 1:
        table = table.contiguous()
    _, indices, _ = ops.table_to_csr(table, selected_block_counts, rows, 1, int(kv_blocks))
    n = min(kv_indices.numel(), indices.numel())
    kv_indices[:n].copy_(indices[:n])


def _raise_no_counterpart(name: str):
    def fn(**kwargs):
        raise NotImplementedError(
            f"{name}: no counterpart on MI355X -- ca_attn_fwd reads the selected cache pages in place, "
            "so the gathered workspace this builds is not needed")
    fn.__name__ = name
    return fn


for _name in ("build_block_table_cuda", "pack_q_for_indexed_prefill_cuda", "compact_keep_blocks_cuda",
              "compact_keep_blocks_cuda_out", "compact_keep_blocks_and_build_table_cuda",
              "compact_keep_blocks_and_build_table_cuda_out", "build_flashinfer_kv_indices_per_query_cuda_out",
              "cache_fill_blocks_to_paged_kv_from_pos_with_rank_cuda",
              "cache_fill_blocks_to_paged_kv_from_pos_with_local_rank_cuda", "cache_fill_from_past_indices_cuda",
              "cache_fill_from_past_indices_compact_cuda", "cache_fill_from_selected_indices_row_tiled_cuda",
              "cache_fill_blocks_to_paged_kv_from_kv_strided_cuda", "cache_fill_current_tail_cuda"):
    globals()[_name] = _raise_no_counterpart(_name)
del _name
