"""Seeded synthetic inputs for the benchmark configurations.

Q, K, V ~ N(0, 1); for every KV head a fixed number of randomly chosen past blocks (never
block 0 nor the local blocks right before the chunk) get ``+plant_scale * u`` added to all
their K rows, u a shared random unit direction -- the "planted high-score blocks" of the
benchmark configurations.  Draw order is fixed, so a seed reproduces the same tensors on
any machine (generation runs on the CPU).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Sequence

import torch

BLOCK = 64
HEAD_DIM = 128
DEFAULT_SEED = 1234  # the reference harness default (eval/chunked_prefill/profile_attention_latency.py:421)

# BASELINE configs 1 and 3's Seer selector as SeerAttnLlamaConfig fields: the AttnGate with
# pooled Q and K both projected per head (Qavg_Kavg, force_double), softmax threshold 5e-3,
# sink block 0 and the 2 local blocks before the chunk.  The reference's own layer has neither
# sink nor local blocks (it forces the last keep_recent_blocks KV blocks); these two fields are
# this build's extension for the benchmark rule.
BASELINE_SEER = dict(seerattn_gate_type="Qavg_Kavg", seerattn_gate_force_double=True,
                     seerattn_compactattn_threshold=5e-3, compactattn_sink_blocks=1, compactattn_local_blocks=2)


@dataclass
class ChunkInputs:
    q: torch.Tensor  # [B, Lq, Hq, 128]
    k: torch.Tensor  # [B, Hkv, Ktot, 128] heads-first, Ktot = max(past) + Lq rounded to cap
    v: torch.Tensor
    past_blocks: List[int]
    kv_cap: int
    planted: List[List[List[int]]] = field(default_factory=list)  # [b][kv head] -> block ids


def make_chunk(batch_past_tokens: Sequence[int], q_len: int, num_q_heads: int, num_kv_heads: int,
               seed: int = DEFAULT_SEED, planted_blocks: int = 8, plant_scale: float = 2.0,
               local_blocks: int = 2, dtype: torch.dtype = torch.bfloat16, kv_cap: int = 0) -> ChunkInputs:
    """Inputs for one chunked-prefill step per request (past lengths may differ)."""
    if q_len % BLOCK:
        raise ValueError("q_len must be a multiple of 64")
    past_blocks = []
    for p in batch_past_tokens:
        if p % BLOCK:
            raise ValueError("past lengths must be multiples of 64")
        past_blocks.append(p // BLOCK)
    B = len(past_blocks)
    qb = q_len // BLOCK
    cap = max(kv_cap, max(past_blocks) + qb)
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    u = torch.randn(HEAD_DIM, generator=g)
    u = u / u.norm()
    q = torch.randn((B, q_len, num_q_heads, HEAD_DIM), generator=g)
    k = torch.randn((B, num_kv_heads, cap * BLOCK, HEAD_DIM), generator=g)
    v = torch.randn((B, num_kv_heads, cap * BLOCK, HEAD_DIM), generator=g)
    planted: List[List[List[int]]] = []
    for b, P in enumerate(past_blocks):
        per_head = []
        lo, hi = 1, P - local_blocks  # candidates exclude the sink block and the local blocks
        for h in range(num_kv_heads):
            if hi - lo >= planted_blocks and planted_blocks > 0:
                ids = (torch.randperm(hi - lo, generator=g)[:planted_blocks] + lo).sort().values.tolist()
            else:
                ids = []
            for blk in ids:
                k[b, h, blk * BLOCK:(blk + 1) * BLOCK] += plant_scale * u
            per_head.append(ids)
        planted.append(per_head)
    # tokens past each request's live length are zeroed (they are never attended)
    for b, P in enumerate(past_blocks):
        live = (P + qb) * BLOCK
        k[b, :, live:] = 0
        v[b, :, live:] = 0
    return ChunkInputs(q.to(dtype), k.to(dtype), v.to(dtype), past_blocks, cap, planted)


def rope_tables(num_rows: int, dim: int = HEAD_DIM, theta: float = 500000.0, stride: int = BLOCK):
    """cos/sin [num_rows, dim] fp32 for positions row*stride (HF rotate_half convention,
    emb = cat(freqs, freqs)); row r is the RoPE of block r's first token."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    pos = torch.arange(num_rows, dtype=torch.float64) * stride
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(torch.float32), emb.sin().to(torch.float32)


def make_chunk_device(past_tokens: int, q_len: int, num_q_heads: int, num_kv_heads: int, device,
                      seed: int = DEFAULT_SEED, planted_blocks: int = 8, plant_scale: float = 2.0,
                      local_blocks: int = 2, kv_cap: int = 0) -> ChunkInputs:
    """Single-request inputs generated on the GPU (large configurations); same structure
    as make_chunk, drawn from a device generator."""
    if q_len % BLOCK or past_tokens % BLOCK:
        raise ValueError("lengths must be multiples of 64")
    P = past_tokens // BLOCK
    qb = q_len // BLOCK
    cap = max(kv_cap, P + qb)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    u = torch.randn(HEAD_DIM, generator=g, device=device)
    u = u / u.norm()
    q = torch.randn((1, q_len, num_q_heads, HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    k = torch.empty((1, num_kv_heads, cap * BLOCK, HEAD_DIM), dtype=torch.bfloat16, device=device)
    v = torch.empty_like(k)
    for h in range(num_kv_heads):  # per head to bound the fp32 temporaries
        k[0, h] = torch.randn((cap * BLOCK, HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
        v[0, h] = torch.randn((cap * BLOCK, HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    planted: List[List[int]] = []
    lo, hi = 1, P - local_blocks
    for h in range(num_kv_heads):
        ids = []
        if hi - lo >= planted_blocks and planted_blocks > 0:
            ids = (torch.randperm(hi - lo, generator=g, device=device)[:planted_blocks] + lo).sort().values.tolist()
        for blk in ids:
            seg = k[0, h, blk * BLOCK:(blk + 1) * BLOCK]
            seg.copy_((seg.float() + plant_scale * u).to(torch.bfloat16))
        planted.append(ids)
    live = (P + qb) * BLOCK
    k[:, :, live:] = 0
    v[:, :, live:] = 0
    return ChunkInputs(q, k, v, [P], cap, [planted])
