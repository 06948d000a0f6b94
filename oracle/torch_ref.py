"""fp32 PyTorch restatement of one compactattn chunk step on the CPU.

TEST INFRASTRUCTURE / CPU BASELINE ONLY: bench.py's ``cpu_baseline`` leg times it (and tests
may use it as a checker); the product package ``compactattention_amd`` never imports it.

One layer-chunk of the path, vectorised over heads with BLAS-backed fp32 GEMMs (the
reference's own path cannot run on a CPU: it needs flash_attn, CUDA and Triton):
  1. cache update: the chunk's K/V concatenated onto the past, as transformers'
     DynamicCache.update does for the reference's layers
     (compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:518-536);
  2. mean-K of the chunk's blocks appended to the per-layer mean-K cache
     (modeling_llama_flashprefill_compactattn.py:121-150);
  3. pooled block scores: mean-pooled Q of each query block against every causal mean-K
     block, times d^-1/2, softmax over the causal key blocks (this path's FlashPrefill
     scores, normalised over key blocks as flashprefill_native_forward.py:365-374);
  4. selection per (Q head, query block) row: the top-k past blocks (torch.topk), the sink
     blocks and the local blocks before the chunk; then the Q-block union, the current chunk
     kept, the GQA union (compact_attn/modules/attention_forward_chunked_dense.py:641-683)
     and ascending block lists (flashinfer_zero_copy_prefill.py:482-510);
  5. attention of every query over its KV row's selected blocks with bottom-right causal
     masking (indexed_dense_prefill_direct_triton.py:91-241 semantics): gather, q k^T,
     softmax, PV.

decoder_layer_step wraps chunk_step in one Llama decoder layer (RMSNorm, q/k/v projections,
rotate_half RoPE, o_proj and the residual, RMSNorm, SwiGLU MLP), the layer the reference's
compactattn models run per chunk (modeling_llama_seerattn_chunked_dense.py:547-938 around the
attention call); bench.py times it for the whole-model (config 3) CPU extrapolation.
"""
from __future__ import annotations

import math
from typing import List, Tuple

import torch

BLOCK = 64


def block_means(x: torch.Tensor) -> torch.Tensor:
    """[B, L, H, D] -> [B, H, L/64, D] fp32 block means."""
    B, L, H, D = x.shape
    return x.float().view(B, L // BLOCK, BLOCK, H, D).mean(dim=2).permute(0, 2, 1, 3).contiguous()


def select_tables(qhat: torch.Tensor, khat: torch.Tensor, past: int, topk: int, sink: int, local: int,
                  scale: float) -> List[torch.Tensor]:
    """qhat [B, Hq, Qb, D], khat [B, Hkv, P+Qb, D] -> per (b, kv head) ascending block ids."""
    B, Hq, Qb, D = qhat.shape
    Hkv, nkb = khat.shape[1], khat.shape[2]
    G = Hq // Hkv
    kq = khat.repeat_interleave(G, dim=1)  # [B, Hq, nkb, D]
    s = torch.matmul(qhat, kq.transpose(-1, -2)) * scale  # [B, Hq, Qb, nkb]
    causal = torch.arange(nkb)[None, :] <= (past + torch.arange(Qb))[:, None]
    s = torch.softmax(s.masked_fill(~causal, float("-inf")), dim=-1)
    keep = torch.zeros((B, Hq, Qb, nkb), dtype=torch.bool)
    if topk > 0 and past > 0:
        idx = torch.topk(s[..., :past], k=min(topk, past), dim=-1).indices
        keep.scatter_(-1, idx, True)
    keep[..., :min(sink, past)] = True
    keep[..., max(past - local, 0):past] = True
    kv = keep.any(dim=2).view(B, Hkv, G, nkb).any(dim=2)  # Q-block then GQA union
    kv[..., past:] = True
    return [torch.nonzero(kv[b, h]).flatten() for b in range(B) for h in range(Hkv)]


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tables: List[torch.Tensor], past: int,
              scale: float) -> torch.Tensor:
    """q [B, Lq, Hq, D] fp32, k/v [B, Hkv, K, D] fp32 heads-first -> out [B, Lq, Hq, D]."""
    B, Lq, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    out = torch.empty_like(q)
    qpos = (past * BLOCK + torch.arange(Lq)).repeat_interleave(G)  # packed rows t*G + g
    ar = torch.arange(BLOCK)
    for b in range(B):
        for h in range(Hkv):
            keys = (tables[b * Hkv + h][:, None] * BLOCK + ar[None, :]).flatten()
            kf = k[b, h].index_select(0, keys)
            vf = v[b, h].index_select(0, keys)
            qf = q[b, :, h * G:(h + 1) * G].reshape(Lq * G, D)
            s = torch.matmul(qf, kf.T) * scale
            s.masked_fill_(keys[None, :] > qpos[:, None], float("-inf"))
            out[b, :, h * G:(h + 1) * G] = torch.matmul(torch.softmax(s, dim=-1), vf).view(Lq, G, D)
    return out


def chunk_step(q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor, k_new: torch.Tensor,
               v_new: torch.Tensor, kmean_past: torch.Tensor, topk: int, sink: int = 1, local: int = 2
               ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, List[torch.Tensor]]:
    """One layer-chunk: q [B, Lq, Hq, D]; past K/V [B, Hkv, P*64, D] heads-first and their
    mean-K [B, Hkv, P, D]; the chunk's K/V [B, Lq, Hkv, D].  Everything fp32.  Returns
    (out, k_all, v_all, kmean_all, tables)."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    past = k_past.shape[2] // BLOCK
    k_all = torch.cat([k_past, k_new.transpose(1, 2)], dim=2)  # DynamicCache.update
    v_all = torch.cat([v_past, v_new.transpose(1, 2)], dim=2)
    kmean_all = torch.cat([kmean_past, block_means(k_new)], dim=2)
    tables = select_tables(block_means(q), kmean_all, past, topk, sink, local, scale)
    out = attention(q, k_all, v_all, tables, past, scale)
    return out, k_all, v_all, kmean_all, tables


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """Llama RMSNorm in fp32: x / sqrt(mean(x^2) + eps) * w."""
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w


def rope(x: torch.Tensor, pos: torch.Tensor, theta: float = 500000.0) -> torch.Tensor:
    """rotate_half RoPE (compact_attn/modules/common.py:29-81 convention): x [B, L, H, D] at
    positions pos [L]."""
    D = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = pos.double()[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], dim=-1).float()[None, :, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], dim=-1).float()[None, :, None, :]
    x1, x2 = x[..., :D // 2], x[..., D // 2:]
    return x * cos + torch.cat([-x2, x1], dim=-1) * sin


def decoder_layer_step(h: torch.Tensor, w: dict, k_past: torch.Tensor, v_past: torch.Tensor,
                       kmean_past: torch.Tensor, num_q_heads: int, num_kv_heads: int, topk: int
                       ) -> torch.Tensor:
    """One Llama decoder layer over a chunk h [B, L, hidden] fp32 whose past K/V (heads-first,
    [B, Hkv, P*64, 128]) and mean-K are cached: the attention is chunk_step's selection and
    sparse attention.  w holds ln1, wq, wk, wv, wo, ln2, wg, wu, wd ([out, in] like nn.Linear)."""
    B, L, _ = h.shape
    D = 128
    pos = k_past.shape[2] + torch.arange(L)
    x = rms_norm(h, w["ln1"])
    q = rope((x @ w["wq"].T).view(B, L, num_q_heads, D), pos)
    k = rope((x @ w["wk"].T).view(B, L, num_kv_heads, D), pos)
    v = (x @ w["wv"].T).view(B, L, num_kv_heads, D)
    out = chunk_step(q, k_past, v_past, k, v, kmean_past, topk)[0]
    h = h + out.reshape(B, L, num_q_heads * D) @ w["wo"].T
    x = rms_norm(h, w["ln2"])
    return h + (torch.nn.functional.silu(x @ w["wg"].T) * (x @ w["wu"].T)) @ w["wd"].T
