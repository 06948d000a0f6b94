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
  - block_size is 64 or 128; a 128-token mean is the token-count-weighted mean of its two
    64-token means (ca_pair_block_summaries), so one 64-token mean-K cache serves both.
A partial last block (a length that is not a multiple of the block size) averages its valid
tokens, as compute_mean_vector does.  The returned tensors are views in the reference's axis
order over the kernels' layouts (mean-K [B, Hkv, Kb, D] underneath, scores [B, Hq, Qb, Kb]
underneath).
"""
from __future__ import annotations

import math

import torch

from .. import ops

BLOCK = 64


def _check_block(block_size: int) -> None:
    if block_size not in (64, 128):
        raise ValueError(f"block_size={block_size}: FlashPrefill scoring runs 64- or 128-token blocks")


def _means64_to(block_size: int, means: torch.Tensor, tokens: int) -> torch.Tensor:
    """[B, H, ceil(tokens/64), D] 64-token means -> means in block_size blocks."""
    if block_size == BLOCK:
        return means
    nb = means.shape[2]
    return ops.pair_block_summaries(means, nb, tokens - BLOCK * (nb - 1))


@torch.no_grad()
def flash_prefill_compute_mean_k(k: torch.Tensor, *, block_size: int) -> torch.Tensor:
    """k [B, K, Hkv, D] bf16 -> fp32 block means viewed as [B, ceil(K/block_size), Hkv, D]."""
    _check_block(block_size)
    B, K, Hkv, D = k.shape
    kb = -(-K // BLOCK)
    mean = torch.empty((B, Hkv, kb, D), dtype=torch.float32, device=k.device)
    ops.cache_fill(k, None, None, None, [0] * B, kb, mean)
    return _means64_to(block_size, mean, K).permute(0, 2, 1, 3)


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
    """q [B, Lq, Hq, D] (the last Lq of key_len positions, starting at a multiple of
    block_size), mean_k [B, Kb, Hkv, D] in block_size blocks -> normalised block scores viewed
    as [B, ceil(Lq/bs), ceil(key_len/bs), Hq] (non-causal entries 0)."""
    _check_block(block_size)
    B, Lq, Hq, D = q.shape
    khat = mean_k_kernel_layout(mean_k)
    Hkv = khat.shape[1]
    kb = -(-key_len // block_size)
    if (key_len - Lq) % block_size or key_len < Lq or kb > khat.shape[2]:
        raise ValueError("the chunk must start at a block boundary and mean_k must cover key_len")
    khat = khat[:, :, :kb].contiguous()
    P = (key_len - Lq) // block_size
    q64 = ops.pool_query(q, [P * (block_size // BLOCK)] * B, (P + -(-Lq // block_size)) * (block_size // BLOCK),
                         num_kv_heads=Hkv)
    qhat = _means64_to(block_size, q64, Lq)
    _, scores = ops.score_select(qhat, khat, 1.0 / math.sqrt(D), ops.Rule(), [P] * B, Hkv, kb, with_scores=True)
    return scores.permute(0, 2, 3, 1)


@torch.no_grad()
def flash_prefill_score_chunked(q: torch.Tensor, k: torch.Tensor, *, block_size: int) -> torch.Tensor:
    mean_k = flash_prefill_compute_mean_k(k, block_size=block_size)
    return flash_prefill_score_chunked_from_mean_k(q, mean_k, key_len=k.shape[1], block_size=block_size)
