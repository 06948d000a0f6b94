"""Shared plumbing of the compactattn operator entry points.

Everything here launches HIP kernels through :mod:`compactattention_amd.ops`; the only
torch GPU ops are tiny layout/glue steps (views, a boolean OR over the query heads of a
group).  There is no CPU or non-HIP fallback.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from .. import ops

BLOCK = 64
HEAD_DIM = 128
COMPACTATTN_VERSION = "mi355x-hip-1"

# the indexed_impl values the reference accepts (attention_forward_chunked_dense.py:2172-2173);
# all of them run the one HIP indexed-attention kernel here
INDEXED_IMPLS = frozenset({
    "fa2_paged", "triton_direct", "fa2_indexed", "fi_paged", "fi_zero_copy", "fi_zero_copy_per_query",
    "fi_zero_copy_subgroup", "cudnn_one_shot",
})


@dataclass
class ChunkGeometry:
    batch: int
    q_len: int
    kv_len: int
    num_q_heads: int
    num_kv_heads: int
    past_blocks: int
    q_blocks: int
    kv_cap: int

    @property
    def group(self) -> int:
        return self.num_q_heads // self.num_kv_heads


def geometry(query_states: torch.Tensor, kv_len: int, num_kv_heads: int, block_size: int) -> ChunkGeometry:
    """The chunk's block geometry.  The chunk starts at a block boundary (kv_len - q_len a
    multiple of 64) and covers Qb = ceil(q_len / 64) blocks; when q_len is not a multiple of
    64 its last block holds q_len % 64 tokens, which the kernels read, pool and attend up to
    kv_len only (a partial block selects and is attended like a whole one)."""
    if block_size != BLOCK:
        raise ValueError(f"block_size={block_size}: this build runs 64-token blocks only")
    if query_states.dim() != 4 or query_states.shape[-1] != HEAD_DIM:
        raise ValueError(f"query_states must be [B, Q, Hq, {HEAD_DIM}]")
    bsz, q_len, num_q_heads, _ = query_states.shape
    if num_q_heads % num_kv_heads:
        raise ValueError(f"num_q_heads={num_q_heads} is not a multiple of num_kv_heads={num_kv_heads}")
    if kv_len < q_len or q_len < 1:
        raise ValueError(f"kv_len={kv_len} < q_len={q_len}")
    if (kv_len - q_len) % BLOCK:
        raise ValueError(f"a chunk of {q_len} queries over {kv_len} keys must start at a 64-token block boundary")
    P = (kv_len - q_len) // BLOCK
    Qb = -(-q_len // BLOCK)
    return ChunkGeometry(bsz, q_len, kv_len, num_q_heads, num_kv_heads, P, Qb, P + Qb)


def starts_mid_block(q_len: int, kv_len: int) -> bool:
    """A chunk that does not start at a 64-token block boundary (decode tokens left the cache
    between two blocks): its queries attend densely (dense_tail) when there are at most 64 of
    them; a longer such chunk raises, as its first query block would straddle two key blocks."""
    if kv_len < q_len:
        raise ValueError(f"kv_len={kv_len} < q_len={q_len}")
    if (kv_len - q_len) % BLOCK == 0:
        return False
    if q_len > BLOCK:
        raise ValueError(f"a chunk of {q_len} queries over {kv_len} keys must start at a 64-token block boundary")
    return True


def dense_tail(query_states: torch.Tensor, K: ops.KV, V: ops.KV, kv_len: int, num_kv_heads: int,
               softmax_scale: Optional[float]) -> torch.Tensor:
    """Queries [B, n, Hq, 128] (n <= 64) at the last n of kv_len positions attend to every key
    before them (bottom-right causal) through the decode kernel, which reads the partial last
    block up to kv_len only -- the reference's dense attention for q_len == 1
    (modeling_llama_seerattn_chunked_dense.py:878-894, flashprefill_prefill.py:903-907)."""
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(HEAD_DIM)
    B = query_states.shape[0]
    return ops.attn_decode(query_states, K, V, [kv_len] * B, scale, -(-kv_len // BLOCK), num_kv_heads)


def kv_layouts(key_states: Optional[torch.Tensor], value_states: Optional[torch.Tensor],
               k_hf: Optional[torch.Tensor], v_hf: Optional[torch.Tensor]) -> Tuple[ops.KV, ops.KV]:
    """Prefer the heads-first cache (zero copy, the reference's fi_zero_copy view); else read
    the seq-first [B, K, Hkv, D] tensors in place through strides."""
    if k_hf is not None and v_hf is not None:
        return ops.KV.heads_first(k_hf), ops.KV.heads_first(v_hf)
    if key_states is None or value_states is None:
        raise ValueError("key_states/value_states or k_hf/v_hf are required")
    return ops.KV.seq_first(key_states), ops.KV.seq_first(value_states)


def check_attention_mask(attention_mask: Optional[torch.Tensor], bsz: int, kv_len: int) -> None:
    """Only the all-ones padding mask of chunked prefill is supported (no partial padding)."""
    if attention_mask is None:
        return
    if attention_mask.dim() != 2 or tuple(attention_mask.shape) != (bsz, kv_len):
        raise ValueError(f"attention_mask must be [B, K] = {(bsz, kv_len)}, got {tuple(attention_mask.shape)}")
    if not bool(attention_mask.to(torch.bool).all()):
        raise ValueError("attention_mask with padded positions is not supported by the compactattn path")


def dense_tables(geo: ChunkGeometry, device) -> Tuple[torch.Tensor, torch.Tensor]:
    return ops.dense_table([geo.past_blocks] * geo.batch, geo.q_len, geo.num_q_heads, geo.num_kv_heads,
                           geo.kv_cap, device)


def attend(query_states: torch.Tensor, K: ops.KV, V: ops.KV, table: torch.Tensor, counts: torch.Tensor,
           geo: ChunkGeometry, softmax_scale: Optional[float]) -> torch.Tensor:
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(HEAD_DIM)
    return ops.attn_fwd(query_states, K, V, table, counts, [geo.past_blocks] * geo.batch, scale, geo.kv_cap,
                        geo.num_kv_heads)


class StageTimer:
    """Event pairs on the launch stream, read once at the end (only when stats are asked for)."""

    def __init__(self, enabled: bool):
        self.enabled = enabled
        self.pairs = []

    def __call__(self, name: str, fn):
        if not self.enabled:
            return fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        out = fn()
        b.record()
        self.pairs.append((name, a, b))
        return out

    def results(self) -> Dict[str, float]:
        if not self.pairs:
            return {}
        self.pairs[-1][2].synchronize()
        return {name: a.elapsed_time(b) for name, a, b in self.pairs}


def table_stats(counts: torch.Tensor, geo: ChunkGeometry, prefix: str) -> Dict[str, float]:
    c = counts.to(torch.float64).cpu()
    past_sel = (c - geo.q_blocks).clamp(min=0)
    density = float(past_sel.mean() / geo.past_blocks) if geo.past_blocks > 0 else 1.0
    return {
        f"{prefix}selected_blocks": float(c.sum()),
        f"{prefix}selected_blocks_past": float(past_sel.sum()),
        f"{prefix}past_density": density,
        f"{prefix}kv_blocks": float(geo.kv_cap),
        f"{prefix}query_blocks": float(geo.q_blocks),
    }
