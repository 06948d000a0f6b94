"""SeerAttention AttnGate on the HIP kernels.

Mirrors compact_attn/prefill_sparse/attn_gate.py (MultiHeadLinear :20-34, AttnGate
:37-222) for the gate this path uses: average pooling of Q and K over 64-token blocks,
per-head 128 -> 128 projections of both (the reference's force_double / Qavg_Kavg form),
block RoPE at each block's first position, q.k^T * hidden^-1/2, causal block mask, softmax
over key blocks.  Pooling + projection + RoPE of the query side run in one kernel
(ca_pool_query), of the key side in the cache-fill kernel (ca_cache_fill summaries), and
the scores in ca_score_select -- all in a fixed fp32 evaluation order.

Weights follow the reference's MultiHeadLinear layout [heads, in, out] and are kept in
fp32.  position_embeddings are (cos, sin) tables [Kb, 128] (or [1, Kb, 128]) holding, in
row kb, the rotary embedding of block kb's first token (the reference's block_rotary_emb
evaluated at position_ids[:, 0::64]).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from .. import ops

BLOCK = 64
HEAD_DIM = 128


class MultiHeadLinear(nn.Module):
    """weight [num_head, in, out]; forward x [B, S, H, in] -> [B, S, H, out] (reference semantics)."""

    def __init__(self, in_channel_size: int, hidden_size: int, num_head: int):
        super().__init__()
        self.in_channel = in_channel_size
        self.hidden_size = hidden_size
        self.num_head = num_head
        self.weight = nn.Parameter(torch.empty(num_head, in_channel_size, hidden_size, dtype=torch.float32))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[2] < self.num_head:
            x = x.repeat_interleave(self.num_head // x.shape[2], dim=2)
        return torch.einsum("bshi,hio->bsho", x, self.weight)


def _rope_rows(position_embeddings):
    if position_embeddings is None:
        return None, None
    cos, sin = position_embeddings
    if cos.dim() == 3:
        if cos.shape[0] != 1:
            raise ValueError("block position embeddings must be shared across the batch")
        cos, sin = cos[0], sin[0]
    return cos.float().contiguous(), sin.float().contiguous()


class AttnGate(nn.Module):
    def __init__(self, block_size: int, in_channel_size: int, hidden_size: int, num_k_head: int, num_q_head: int,
                 q_pooling_funcs=("avg",), k_pooling_funcs=("avg",), force_double: bool = True,
                 use_flash_rope: bool = False, kv_group_aware_query: bool = False):
        super().__init__()
        if block_size != BLOCK:
            raise ValueError("AttnGate block_size must be 64")
        if in_channel_size != HEAD_DIM or hidden_size != HEAD_DIM:
            raise ValueError("AttnGate runs 128-dim heads and a 128-dim gate hidden size")
        if tuple(q_pooling_funcs) != ("avg",) or tuple(k_pooling_funcs) != ("avg",):
            raise ValueError("only average pooling (gate type Qavg_Kavg) is implemented")
        if not force_double or kv_group_aware_query:
            raise ValueError("the gate projects both sides per head (force_double=True, per-Q-head query)")
        if num_q_head % num_k_head:
            raise ValueError(f"num_q_head ({num_q_head}) must be divisible by num_k_head ({num_k_head}).")
        del use_flash_rope
        self.block_size = block_size
        self.hidden_size = hidden_size
        self.num_k_head = num_k_head
        self.num_q_head = num_q_head
        self.num_key_value_groups = num_q_head // num_k_head
        self.scale = hidden_size ** -0.5
        self.mask_linear_q = MultiHeadLinear(in_channel_size, hidden_size, num_q_head)
        self.mask_linear_k = MultiHeadLinear(in_channel_size, hidden_size, num_k_head)

    def reset_parameters(self, initializer_range: float = 0.02, generator: Optional[torch.Generator] = None):
        with torch.no_grad():
            for lin in (self.mask_linear_q, self.mask_linear_k):
                w = torch.randn(lin.weight.shape, generator=generator, dtype=torch.float32) * initializer_range
                lin.weight.copy_(w.to(lin.weight.device))

    # -- the kernels' building blocks --------------------------------------------------------
    @torch.no_grad()
    def compress_query_blocks(self, q: torch.Tensor, first_block: int = 0, position_embeddings=None) -> torch.Tensor:
        """q [B, L, Hq, 128] bf16 -> projected (and rotated) block queries [B, Hq, L/64, 128] fp32."""
        cos, sin = _rope_rows(position_embeddings)
        B, L = q.shape[:2]
        cap = first_block + L // BLOCK
        return ops.pool_query(q, [first_block] * B, cap, gate_wq=self.mask_linear_q.weight.detach().contiguous(),
                              rope_cos=cos, rope_sin=sin, num_kv_heads=self.num_k_head)

    @torch.no_grad()
    def compress_key_blocks(self, k: torch.Tensor, out: Optional[torch.Tensor] = None, first_block: int = 0,
                            position_embeddings=None) -> torch.Tensor:
        """k [B, L, Hkv, 128] bf16 -> projected (and rotated) block keys written into out
        [B, Hkv, cap, 128] fp32 at blocks first_block.. (allocated when None)."""
        cos, sin = _rope_rows(position_embeddings)
        B, L, Hkv, _ = k.shape
        cap = out.shape[2] if out is not None else first_block + L // BLOCK
        if out is None:
            out = torch.zeros((B, Hkv, cap, HEAD_DIM), dtype=torch.float32, device=k.device)
        ops.cache_fill(k, None, None, None, [first_block] * B, cap, None,
                       gate_wk=self.mask_linear_k.weight.detach().contiguous(), rope_cos=cos, rope_sin=sin,
                       kgate=out)
        return out

    @torch.no_grad()
    def forward(self, q: torch.Tensor, k: torch.Tensor, attention_mask=None, position_embeddings=None,
                use_softmax: bool = True) -> Optional[torch.Tensor]:
        """q [B, Lq, Hq, 128] (the last Lq positions), k [B, K, Hkv, 128] (all positions) ->
        gate scores [B, Hq, Qb, Kb] fp32 (softmax over causal key blocks, others 0).

        attention_mask, when given, must be the causal block mask the path applies itself."""
        del attention_mask
        if not use_softmax:
            raise ValueError("the gate scores are produced normalised (use_softmax=True)")
        B, Lq = q.shape[:2]
        if Lq == 1:
            return None
        K = k.shape[1]
        kb = K // BLOCK
        P = (K - Lq) // BLOCK
        kgate = self.compress_key_blocks(k, first_block=0, position_embeddings=position_embeddings)
        qgate = self.compress_query_blocks(q, first_block=P, position_embeddings=position_embeddings)
        _, scores = ops.score_select(qgate, kgate, self.scale, ops.Rule(), [P] * B, self.num_k_head, kb,
                                     with_scores=True)
        return scores
