"""FlashPrefill block summaries and scores on the HIP kernels.

Mirrors compact_attn/flashprefill_vendor/flashprefill_native_forward.py:
  flash_prefill_compute_mean_k            (:505-538)
  flash_prefill_score_chunked_from_mean_k (:541-586)
  flash_prefill_score_chunked             (:589-602)
Deliberate differences (all documented in the build's design notes):
  - mean-K is kept in fp32 (the reference stores it in the K dtype);
  - scores are the softmax over causal key blocks of the pooled logits
    mean(Q_qb) . mean(K_kb) / sqrt(d) (the reference accumulates per-token exp2 mass of
    q_t . mean(K_kb)); both are [B, Qb, Kb, Hq] fp32 probabilities summing to one over kb;
  - block_size is 64.
The returned tensors are views in the reference's axis order over the kernels' layouts
(mean-K [B, Hkv, Kb, D] underneath, scores [B, Hq, Qb, Kb] underneath).
"""
from __future__ import annotations

import math

import torch

from .. import ops

BLOCK = 64


def _check_block(block_size: int) -> None:
    if block_size != BLOCK:
        raise ValueError(f"block_size={block_size}: this build runs 64-token blocks only")


@torch.no_grad()
def flash_prefill_compute_mean_k(k: torch.Tensor, *, block_size: int) -> torch.Tensor:
    """k [B, K, Hkv, D] bf16 -> fp32 block means viewed as [B, Kb, Hkv, D]."""
    _check_block(block_size)
    B, K, Hkv, D = k.shape
    if K % BLOCK:
        raise ValueError(f"key length {K} must be a multiple of {BLOCK}")
    kb = K // BLOCK
    mean = torch.empty((B, Hkv, kb, D), dtype=torch.float32, device=k.device)
    ops.cache_fill(k, None, None, None, [0] * B, kb, mean)
    return mean.permute(0, 2, 1, 3)


def mean_k_kernel_layout(mean_k: torch.Tensor) -> torch.Tensor:
    """[B, Kb, Hkv, D] (any dtype/strides) -> contiguous fp32 [B, Hkv, Kb, D] (no copy when the
    input is a view returned by flash_prefill_compute_mean_k)."""
    m = mean_k.permute(0, 2, 1, 3)
    if m.dtype != torch.float32:
        m = m.float()
    return m.contiguous()


@torch.no_grad()
def flash_prefill_score_chunked_from_mean_k(q: torch.Tensor, mean_k: torch.Tensor, *, key_len: int,
                                            block_size: int) -> torch.Tensor:
    """q [B, Lq, Hq, D] (the last Lq of key_len positions), mean_k [B, Kb, Hkv, D] ->
    normalised block scores viewed as [B, Qb, Kb, Hq] (non-causal entries 0)."""
    _check_block(block_size)
    B, Lq, Hq, D = q.shape
    khat = mean_k_kernel_layout(mean_k)
    Hkv, kb = khat.shape[1], khat.shape[2]
    if key_len % BLOCK or Lq % BLOCK or key_len // BLOCK > kb:
        raise ValueError("key_len and q_len must be block aligned and covered by mean_k")
    P = (key_len - Lq) // BLOCK
    qhat = ops.pool_query(q, [P] * B, kb, num_kv_heads=Hkv)
    _, scores = ops.score_select(qhat, khat, 1.0 / math.sqrt(D), ops.Rule(), [P] * B, Hkv, kb, with_scores=True)
    return scores.permute(0, 2, 3, 1)


@torch.no_grad()
def flash_prefill_score_chunked(q: torch.Tensor, k: torch.Tensor, *, block_size: int) -> torch.Tensor:
    mean_k = flash_prefill_compute_mean_k(k, block_size=block_size)
    return flash_prefill_score_chunked_from_mean_k(q, mean_k, key_len=k.shape[1], block_size=block_size)
