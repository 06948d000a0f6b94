"""SeerAttention AttnGate on the HIP kernels.

Mirrors compact_attn/prefill_sparse/attn_gate.py (MultiHeadLinear :20-34, AttnGate
:37-222, the generated gate classes :233-278) for every gate type the reference builds:
  - Q and K pooled over 64-token blocks by any non-empty subset of (max, min, avg), the
    pooled vectors concatenated in that order (C pools -> C*128 inputs);
  - projections (the reference's three cases, :74-86):
      kv_group_aware_query: W_q [Hkv, G*Cq*128, 128] over the concatenated group, W_k
                            [Hkv, Ck*128, 128]; scores per KV head;
      Cq > 1, hidden != in or force_double: W_q [Hq, Cq*128, 128], W_k [Hkv, Ck*128, 128];
      otherwise (the default Qavg_K*): no query projection, W_k [Hq, Ck*128, 128] on the
                            K blocks repeated to the Q heads (MultiHeadLinear's repeat, :30-33);
  - block RoPE at each block's first position, q.k^T * hidden^-1/2, causal block mask,
    softmax over key blocks.
Query pooling + projection + RoPE run in one kernel (ca_gate_query_summaries), the key side
in another (ca_gate_key_summaries, also used for the gate K-block cache), the scores in
ca_score_select -- all in a fixed fp32 evaluation order.

Weights follow the reference's MultiHeadLinear layout [heads, in, out] (checkpoint key
names attn_gate.mask_linear_q.weight / mask_linear_k.weight) and are kept in fp32.
position_embeddings are (cos, sin) tables [Kb, 128] (or [1, Kb, 128]) holding, in row kb,
the rotary embedding of block kb's first token (the reference's block_rotary_emb evaluated
at position_ids[:, 0::64]).
"""
from __future__ import annotations

from itertools import combinations
from typing import Dict, Optional, Sequence, Tuple

import torch
from torch import nn

from .. import ops

BLOCK = 64
HEAD_DIM = 128
POOL_TYPES = ("max", "min", "avg")


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


def _pool_names(funcs) -> Tuple[str, ...]:
    names = []
    for f in funcs:
        name = f if isinstance(f, str) else getattr(f, "pool_name", None)
        if name not in POOL_TYPES:
            raise ValueError(f"unknown pooling function {f!r}; use 'max', 'min' or 'avg'")
        names.append(name)
    return tuple(names)


class AttnGate(nn.Module):
    def __init__(self, block_size: int, in_channel_size: int, hidden_size: int, num_k_head: int, num_q_head: int,
                 q_pooling_funcs=("avg",), k_pooling_funcs=("avg",), force_double: bool = False,
                 use_flash_rope: bool = False, kv_group_aware_query: bool = False):
        super().__init__()
        if block_size != BLOCK:
            raise ValueError("AttnGate block_size must be 64")
        if in_channel_size != HEAD_DIM or hidden_size != HEAD_DIM:
            raise ValueError("AttnGate runs 128-dim heads and a 128-dim gate hidden size")
        if num_q_head % num_k_head:
            raise ValueError(f"num_q_head ({num_q_head}) must be divisible by num_k_head ({num_k_head}).")
        del use_flash_rope  # both RoPE forms (rotate_half and flash's non-interleaved) are the same formula
        self.block_size = block_size
        self.in_channel = in_channel_size
        self.hidden_size = hidden_size
        self.num_k_head = num_k_head
        self.num_q_head = num_q_head
        self.num_key_value_groups = num_q_head // num_k_head
        self.kv_group_aware_query = bool(kv_group_aware_query)
        self.q_pooling_funcs = _pool_names(q_pooling_funcs)
        self.k_pooling_funcs = _pool_names(k_pooling_funcs)
        self.q_pools = ops.pool_bits(self.q_pooling_funcs)
        self.k_pools = ops.pool_bits(self.k_pooling_funcs)
        self.scale = hidden_size ** -0.5
        self.q_dup_size = len(self.q_pooling_funcs)
        self.k_dup_size = len(self.k_pooling_funcs)
        q_in = in_channel_size * self.q_dup_size
        k_in = in_channel_size * self.k_dup_size
        G = self.num_key_value_groups
        if self.kv_group_aware_query:
            self.mask_linear_q = MultiHeadLinear(G * q_in, hidden_size, num_k_head)
            self.mask_linear_k = MultiHeadLinear(k_in, hidden_size, num_k_head)
        elif self.q_dup_size > 1 or hidden_size != in_channel_size or force_double:
            self.mask_linear_q = MultiHeadLinear(q_in, hidden_size, num_q_head)
            self.mask_linear_k = MultiHeadLinear(k_in, hidden_size, num_k_head)
        else:  # a single linear layer on the K side, per Q head
            self.mask_linear_q = None
            self.mask_linear_k = MultiHeadLinear(k_in, hidden_size, num_q_head)

    # -- head counts of the summaries ---------------------------------------------------------
    @property
    def query_heads(self) -> int:
        """Heads of the query summaries (and of the gate scores)."""
        return self.num_k_head if self.kv_group_aware_query else self.num_q_head

    @property
    def key_heads(self) -> int:
        """Heads of the key summaries (the gate K-block cache)."""
        return self.mask_linear_k.num_head

    def reset_parameters(self, initializer_range: float = 0.02, generator: Optional[torch.Generator] = None):
        with torch.no_grad():
            for lin in (self.mask_linear_q, self.mask_linear_k):
                if lin is None:
                    continue
                w = torch.randn(lin.weight.shape, generator=generator, dtype=torch.float32) * initializer_range
                lin.weight.copy_(w.to(lin.weight.device))

    def reset_query_branch_parameters(self, initializer_range: float) -> None:
        if self.mask_linear_q is None:
            return
        with torch.no_grad():
            self.mask_linear_q.weight.data.normal_(mean=0.0, std=initializer_range)

    # -- the kernels' building blocks --------------------------------------------------------
    @torch.no_grad()
    def compress_query_blocks(self, q: torch.Tensor, first_block: int = 0, position_embeddings=None,
                              kv_cap: Optional[int] = None) -> torch.Tensor:
        """q [B, L, Hq, 128] bf16 -> pooled (projected, rotated) block queries
        [B, query_heads, L/64, 128] fp32; block n sits at absolute block id first_block + n."""
        cos, sin = _rope_rows(position_embeddings)
        B, L = q.shape[:2]
        cap = kv_cap if kv_cap is not None else first_block + L // BLOCK
        wq = self.mask_linear_q.weight.detach().contiguous() if self.mask_linear_q is not None else None
        return ops.gate_query_summaries(q, [first_block] * B, cap, self.q_pools, wq, self.num_k_head, rope_cos=cos,
                                        rope_sin=sin)

    @torch.no_grad()
    def compress_key_blocks(self, k: torch.Tensor, out: Optional[torch.Tensor] = None, first_block: int = 0,
                            position_embeddings=None) -> torch.Tensor:
        """k [B, L, Hkv, 128] bf16 -> pooled, projected (and rotated) block keys written into
        out [B, key_heads, cap, 128] fp32 at blocks first_block.. (allocated when None)."""
        cos, sin = _rope_rows(position_embeddings)
        B, L, Hkv, _ = k.shape
        cap = out.shape[2] if out is not None else first_block + L // BLOCK
        if out is None:
            out = torch.zeros((B, self.key_heads, cap, HEAD_DIM), dtype=torch.float32, device=k.device)
        ops.gate_key_summaries(k, [first_block] * B, cap, self.k_pools,
                               self.mask_linear_k.weight.detach().contiguous(), out, num_q_heads=self.num_q_head,
                               rope_cos=cos, rope_sin=sin)
        return out

    @torch.no_grad()
    def forward(self, q: torch.Tensor, k: torch.Tensor, attention_mask=None, position_embeddings=None,
                use_softmax: bool = True) -> Optional[torch.Tensor]:
        """q [B, Lq, Hq, 128] (the last Lq positions), k [B, K, Hkv, 128] (all positions) ->
        gate scores [B, query_heads, Qb, Kb] fp32 (softmax over causal key blocks, others 0).

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
        qgate = self.compress_query_blocks(q, first_block=P, position_embeddings=position_embeddings, kv_cap=kb)
        _, scores = ops.score_select(qgate, kgate, self.scale, ops.Rule(), [P] * B, self.key_heads, kb,
                                     with_scores=True)
        return scores


def parse_gate_type(gate_type: str) -> Tuple[Tuple[str, ...], Tuple[str, ...]]:
    """'Qavg_Kmaxminavg' -> (('avg',), ('max', 'min', 'avg')) (the reference's class names)."""
    try:
        qpart, kpart = gate_type.split("_")
        assert qpart[0] == "Q" and kpart[0] == "K"
    except (ValueError, AssertionError, IndexError):
        raise ValueError(f"gate type {gate_type!r} is not of the form Q<pools>_K<pools>") from None

    def names(s: str) -> Tuple[str, ...]:
        out = []
        while s:
            for nm in POOL_TYPES:
                if s.startswith(nm):
                    out.append(nm)
                    s = s[len(nm):]
                    break
            else:
                raise ValueError(f"gate type {gate_type!r}: unknown pooling name at {s!r}")
        return tuple(out)

    return names(qpart[1:]), names(kpart[1:])


def gate_key_heads(gate_type: str, force_double: bool, kv_group_aware_query: bool, num_q_head: int,
                   num_k_head: int) -> int:
    """Heads of a gate's key summaries: the query count when the gate has no query projection
    (one query pool, no force_double, not kv-group-aware: attn_gate.py:84-86), else the KV count."""
    q_names, _ = parse_gate_type(gate_type)
    if not kv_group_aware_query and len(q_names) == 1 and not force_double:
        return num_q_head
    return num_k_head


def _gate_class(q_names: Sequence[str], k_names: Sequence[str]):
    class_name = f"Q{''.join(q_names)}_K{''.join(k_names)}"

    class NewAttnGate(AttnGate):
        def __init__(self, block_size, in_channel_size, hidden_size, num_k_head, num_q_head, force_double=False,
                     use_flash_rope=False, kv_group_aware_query=False):
            super().__init__(block_size, in_channel_size, hidden_size, num_k_head, num_q_head,
                             q_pooling_funcs=tuple(q_names), k_pooling_funcs=tuple(k_names),
                             force_double=force_double, use_flash_rope=use_flash_rope,
                             kv_group_aware_query=kv_group_aware_query)

    NewAttnGate.__name__ = class_name
    NewAttnGate.__qualname__ = class_name
    return class_name, NewAttnGate


def generate_combinations() -> Dict[str, type]:
    """Every Q{pools}_K{pools} gate class, as the reference generates them (attn_gate.py:265-278)."""
    classes = {}
    for nq in range(1, 4):
        for nk in range(1, 4):
            for qc in combinations(POOL_TYPES, nq):
                for kc in combinations(POOL_TYPES, nk):
                    name, cls = _gate_class(qc, kc)
                    classes[name] = cls
    return classes


ATTNGATE_CLASSES = generate_combinations()
