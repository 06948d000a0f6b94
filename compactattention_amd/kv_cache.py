"""Paged KV cache owned by the compactattn path.

Replaces transformers' DynamicCache concatenation for the chunked-prefill layers
(compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:518-536 and the
heads-first _hf cache, modeling_llama_seerattn_chunked_dense_hf.py:59-82) plus the per-layer
mean-K cache of the FlashPrefill model (modeling_llama_flashprefill_compactattn.py:121-150)
and the gate K-block cache of the Seer model (modeling_llama_seerattn_chunked_dense.py:
398-478).

Layout (one layer): K and V are heads-first [B, Hkv, cap*64, 128] bf16, i.e. 64-token
pages with page id (b*Hkv + h)*cap + kb -- exactly the k_hf/v_hf view the reference's
zero-copy path reads.  Block summaries are fp32 [B, Hkv, cap, 128]: kmean (FlashPrefill
scoring) and, when a gate is attached, kgate (projected + rotated mean-K of the AttnGate).
Appends go through the cache-fill kernel, which writes the chunk's pages and its
summaries in one pass; nothing is ever re-copied.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ops

BLOCK = 64
HEAD_DIM = 128


class PagedKVCache:
    def __init__(self, batch: int, num_kv_heads: int, max_tokens: int, device, with_kmean: bool = True,
                 with_kgate: bool = False):
        if max_tokens % BLOCK:
            raise ValueError("max_tokens must be a multiple of 64")
        self.batch = batch
        self.num_kv_heads = num_kv_heads
        self.cap = max_tokens // BLOCK
        self.device = torch.device(device)
        self.k = torch.zeros((batch, num_kv_heads, self.cap * BLOCK, HEAD_DIM), dtype=torch.bfloat16, device=device)
        self.v = torch.zeros_like(self.k)
        self.kmean = (torch.zeros((batch, num_kv_heads, self.cap, HEAD_DIM), dtype=torch.float32, device=device)
                      if with_kmean else None)
        self.kgate = (torch.zeros((batch, num_kv_heads, self.cap, HEAD_DIM), dtype=torch.float32, device=device)
                      if with_kgate else None)
        self.length = 0  # tokens stored per request (all requests advance together)

    @property
    def past_blocks(self) -> int:
        return self.length // BLOCK

    def layouts(self) -> Tuple[ops.KV, ops.KV]:
        return ops.KV.heads_first(self.k), ops.KV.heads_first(self.v)

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, gate_wk: Optional[torch.Tensor] = None,
               rope_cos: Optional[torch.Tensor] = None, rope_sin: Optional[torch.Tensor] = None) -> int:
        """Append [B, L, Hkv, 128] bf16 K/V (L a multiple of 64); returns the number of past
        blocks before the append."""
        B, L, Hkv, _ = k_new.shape
        if B != self.batch or Hkv != self.num_kv_heads:
            raise ValueError("k_new does not match the cache's batch / KV heads")
        if L % BLOCK:
            raise ValueError("appended chunks must be multiples of 64 tokens")
        if self.length % BLOCK:
            raise ValueError("chunked prefill cannot follow decode steps that left a partial block")
        if self.length + L > self.cap * BLOCK:
            raise ValueError(f"cache capacity {self.cap * BLOCK} tokens exceeded")
        if gate_wk is not None and self.kgate is None:
            raise ValueError("cache built without a gate-K summary buffer")
        past = self.past_blocks
        K, V = self.layouts()
        ops.cache_fill(k_new, v_new, K, V, [past] * B, self.cap, self.kmean, gate_wk=gate_wk, rope_cos=rope_cos,
                       rope_sin=rope_sin, kgate=self.kgate if gate_wk is not None else None)
        self.length += L
        return past

    def append_tokens(self, k_new: torch.Tensor, v_new: torch.Tensor) -> int:
        """Decode append: [B, L, Hkv, 128] bf16 K/V (any L) at the current length, which need
        not be block-aligned; returns the length before the append.  Block summaries are
        not maintained for these tokens, so chunked prefill cannot follow decode steps
        (append() rejects a length that is not a multiple of 64)."""
        B, L, Hkv, _ = k_new.shape
        if B != self.batch or Hkv != self.num_kv_heads:
            raise ValueError("k_new does not match the cache's batch / KV heads")
        if self.length + L > self.cap * BLOCK:
            raise ValueError(f"cache capacity {self.cap * BLOCK} tokens exceeded")
        start = self.length
        self.k[:, :, start:start + L].copy_(k_new.transpose(1, 2))
        self.v[:, :, start:start + L].copy_(v_new.transpose(1, 2))
        self.length += L
        return start

    def k_hf(self) -> torch.Tensor:
        return self.k[:, :, :self.length]

    def v_hf(self) -> torch.Tensor:
        return self.v[:, :, :self.length]

    def reset(self) -> None:
        self.length = 0
