"""Llama decoder pieces shared by the compactattn models, plus the per-layer paged cache.

The reference builds its compactattn models on transformers' Llama classes
(compact_attn/prefill_sparse/llama/modeling_llama_seerattn.py: SeerAttnLlamaDecoderLayer,
SeerAttnLlamaModel, SeerAttnLlamaForCausalLM) with a DynamicCache.  Here the decoder is
written directly on PyTorch-ROCm (projections are hipBLASLt GEMMs through nn.Linear), the
attention modules run the HIP compactattn kernels, and the cache is a set of
preallocated per-layer PagedKVCache objects, so a chunk's K/V is appended in place
instead of re-concatenated.

Shapes: hidden states [B, L, hidden]; Q/K/V [B, L, heads, 128].  Rotary tables are fp32,
computed once for every position ([max_positions, 128]); the block tables the gate uses
take the row of each block's first token (modeling_llama_seerattn.py:896-897).
"""
from __future__ import annotations

from contextlib import contextmanager
from typing import List, Optional, Sequence, Tuple, Type

import torch
import torch.nn.functional as F
from torch import nn

from ... import ops
from ...kv_cache import PagedKVCache
from .configuration_llama_seerattn import SeerAttnLlamaConfig

BLOCK = 64


class FusedProjections:
    """One GEMM for several bias-free nn.Linear modules of the owner that read the same
    input (q/k/v, gate/up).  Their weights are re-seated as row blocks (views) of one
    contiguous [sum(out_features), in_features] store, so the modules, their parameters and
    their state_dict keys stay as they are and nothing is duplicated.  The modules are looked
    up by name on every call: if one was replaced, re-created or moved (Module.to), the store
    no longer backs it and the modules are called one by one; ``refuse()`` re-seats them."""

    def __init__(self, owner: nn.Module, names: Sequence[str]):
        self.owner = owner
        self.names = tuple(names)
        self.refuse()

    def refuse(self) -> None:
        mods = [getattr(self.owner, n) for n in self.names]
        self.sizes = [m.out_features for m in mods]
        self.store = torch.cat([m.weight.detach() for m in mods], 0)
        off = 0
        for m, n in zip(mods, self.sizes):
            m.weight = nn.Parameter(self.store[off:off + n], requires_grad=m.weight.requires_grad)
            off += n

    def intact(self) -> bool:
        row_bytes = self.store.shape[1] * self.store.element_size()
        off = 0
        for name, n in zip(self.names, self.sizes):
            m = getattr(self.owner, name)
            w = m.weight
            if (m.bias is not None or w.shape != (n, self.store.shape[1]) or w.dtype != self.store.dtype
                    or w.data_ptr() != self.store.data_ptr() + off * row_bytes):
                return False
            off += n
        return True

    def __call__(self, x: torch.Tensor) -> Tuple[torch.Tensor, ...]:
        if self.intact():
            return F.linear(x, self.store).split(self.sizes, dim=-1)
        return tuple(getattr(self.owner, n)(x) for n in self.names)


class LlamaRMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float, device=None, dtype=torch.bfloat16):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))
        self.eps = eps

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None):
        """transformers' LlamaRMSNorm formula (fp32 statistics, bf16 normalised value times
        the weight) in one HIP kernel.  With ``residual`` the norm is taken of
        bf16(x + residual) and (sum, normed) is returned: the decoder's residual add fused
        into the norm that follows it."""
        return ops.rmsnorm(x, self.weight, self.eps, residual=residual)


class LlamaMLP(nn.Module):
    def __init__(self, config: SeerAttnLlamaConfig, device=None, dtype=torch.bfloat16):
        super().__init__()
        kw = dict(bias=False, device=device, dtype=dtype)
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, **kw)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, **kw)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, **kw)
        self.gate_up = FusedProjections(self, ("gate_proj", "up_proj"))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # one GEMM for gate and up; bf16(silu(gate)) * up in one HIP kernel (F.silu(gate) * up,
        # rounded alike)
        gate, up = self.gate_up(x)
        return self.down_proj(ops.swiglu(gate, up))


class LlamaRotaryEmbedding(nn.Module):
    """cos/sin tables [max_positions, head_dim] (fp32) with the rotate_half layout."""

    def __init__(self, config: SeerAttnLlamaConfig, device=None):
        super().__init__()
        d = config.head_dim
        inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
        pos = torch.arange(config.max_position_embeddings, dtype=torch.float64)
        freqs = torch.outer(pos, inv_freq)
        emb = torch.cat([freqs, freqs], dim=-1)
        self.register_buffer("cos", emb.cos().float().to(device), persistent=False)
        self.register_buffer("sin", emb.sin().float().to(device), persistent=False)
        self.register_buffer("block_cos", self.cos[::BLOCK].contiguous(), persistent=False)
        self.register_buffer("block_sin", self.sin[::BLOCK].contiguous(), persistent=False)

    def tokens(self, start: int, length: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if start + length > self.cos.shape[0]:
            raise ValueError(f"positions up to {start + length} exceed max_position_embeddings {self.cos.shape[0]}")
        return self.cos[start:start + length], self.sin[start:start + length]

    def blocks(self) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.block_cos, self.block_sin


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """q [B, L, Hq, D], k [B, L, Hkv, D], cos/sin [L, D] fp32 -> rotated (input dtype).
    Same formula as the reference's apply_rotary_pos_emb (modules/common.py:29-81),
    evaluated in fp32."""
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    qf, kf = q.float(), k.float()
    return (qf * c + rotate_half(qf) * s).to(q.dtype), (kf * c + rotate_half(kf) * s).to(k.dtype)


@contextmanager
def event_span(sink: Optional[list]):
    """Records a (start, end) pair of timing events on the current stream around the block
    into ``sink`` when it is a list (no-op for None): the attention share of a model run."""
    if sink is None:
        yield
        return
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    yield
    end.record()
    sink.append((start, end))


def project_qkv(attn: nn.Module, hidden_states: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """q [B, L, Hq, D], k and v [B, L, Hkv, D] (strided views of one GEMM's output when the
    module's projections are fused)."""
    B, L, _ = hidden_states.shape
    q, k, v = attn.qkv(hidden_states)
    return (q.view(B, L, attn.num_heads, attn.head_dim), k.view(B, L, attn.num_key_value_heads, attn.head_dim),
            v.view(B, L, attn.num_key_value_heads, attn.head_dim))


def rope_qk(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor
            ) -> Tuple[torch.Tensor, torch.Tensor]:
    """apply_rotary_pos_emb through the HIP rotary kernel (bit-identical results)."""
    cos, sin = cos.float().contiguous(), sin.float().contiguous()
    return ops.rope(q, cos, sin), ops.rope(k, cos, sin)


def dense_decode_forward(attn: nn.Module, hidden_states: torch.Tensor, position_embeddings, cache: PagedKVCache):
    """Decode step(s) of a compactattn attention module: up to 64 new tokens per request
    attend densely to the whole cache (the reference routes q_len == 1 to dense attention,
    compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:878-894).
    K/V of the new tokens are appended at the cache's current length."""
    B, L, _ = hidden_states.shape
    if L > BLOCK:
        raise ValueError(f"decode steps take at most {BLOCK} tokens per call (got {L})")
    q, k, v = project_qkv(attn, hidden_states)
    cos, sin = position_embeddings
    query_states, key_states = rope_qk(q, k, cos, sin)
    cache.append_tokens(key_states, v)
    K, V = cache.layouts()
    out = ops.attn_decode(query_states.contiguous(), K, V, [cache.length] * B, attn.scaling, cache.cap,
                          attn.num_key_value_heads)
    return attn.o_proj(out.reshape(B, L, -1))


def is_decode_step(hidden_states: torch.Tensor, cache: PagedKVCache) -> bool:
    """One new token, or a cache already past a block boundary (decode steps left it inside a
    block), is a dense decode step; any other call of two or more tokens is a chunk that
    selects (the reference's chunked_prefill = q_len > 1 and kv_len > q_len,
    compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:622-640),
    whatever its length: a chunk that is not a multiple of 64 tokens ends in a partial block."""
    return hidden_states.shape[1] == 1 or cache.length % BLOCK != 0


class ChunkedPrefillCache:
    """One PagedKVCache per layer (all layers advance together)."""

    def __init__(self, config: SeerAttnLlamaConfig, batch: int, max_tokens: int, device, with_kmean: bool,
                 with_kgate: bool):
        from ..attn_gate import gate_key_heads

        max_tokens = -(-max_tokens // BLOCK) * BLOCK
        kgate_heads = gate_key_heads(config.seerattn_gate_type, config.seerattn_gate_force_double,
                                     config.seerattn_compactattn_kv_group_aware_gate, config.num_attention_heads,
                                     config.num_key_value_heads)
        self.layers: List[PagedKVCache] = [
            PagedKVCache(batch, config.num_key_value_heads, max_tokens, device, with_kmean=with_kmean,
                         with_kgate=with_kgate, kgate_heads=kgate_heads)
            for _ in range(config.num_hidden_layers)
        ]
        # pages for max_tokens up front, so a prefill of that length maps nothing on the way;
        # a longer sequence grows the pool and the page tables on demand
        for layer in self.layers:
            layer.reserve(max_tokens)

    def layer(self, idx: int) -> PagedKVCache:
        return self.layers[idx]

    def get_seq_length(self) -> int:
        return self.layers[0].length

    def reset(self) -> None:
        """Start a new sequence in the same pages (pages shared by a fork are released)."""
        for c in self.layers:
            c.reset(keep_pages=True)


class CompactAttnLlamaDecoderLayer(nn.Module):
    def __init__(self, config: SeerAttnLlamaConfig, layer_idx: int, attn_cls: Type[nn.Module], device=None):
        super().__init__()
        self.self_attn = attn_cls(config, layer_idx, device=device)
        self.mlp = LlamaMLP(config, device=device)
        self.input_layernorm = LlamaRMSNorm(config.hidden_size, config.rms_norm_eps, device=device)
        self.post_attention_layernorm = LlamaRMSNorm(config.hidden_size, config.rms_norm_eps, device=device)

    def forward(self, hidden_states: torch.Tensor, position_embeddings, block_position_embeddings,
                past_key_value: ChunkedPrefillCache, residual: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
        """The layer's input is residual + hidden_states (hidden_states alone when residual
        is None); returns (mlp_out, residual) whose sum is the layer's output.  Each residual
        add is fused into the norm that follows it, with the same bf16 rounding as the
        unfused ``residual + h``."""
        if residual is None:
            residual, h = hidden_states, self.input_layernorm(hidden_states)
        else:
            residual, h = self.input_layernorm(hidden_states, residual)
        h = self.self_attn(h, position_embeddings, None, past_key_value=past_key_value,
                           block_position_embeddings=block_position_embeddings)[0]
        residual, h = self.post_attention_layernorm(h, residual)
        return self.mlp(h), residual


class CompactAttnLlamaModel(nn.Module):
    def __init__(self, config: SeerAttnLlamaConfig, attn_cls: Type[nn.Module], device=None):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, device=device, dtype=torch.bfloat16)
        self.layers = nn.ModuleList([CompactAttnLlamaDecoderLayer(config, i, attn_cls, device=device)
                                     for i in range(config.num_hidden_layers)])
        self.norm = LlamaRMSNorm(config.hidden_size, config.rms_norm_eps, device=device)
        self.rotary_emb = LlamaRotaryEmbedding(config, device=device)

    def forward(self, input_ids: torch.Tensor, past_key_values: ChunkedPrefillCache) -> torch.Tensor:
        start = past_key_values.get_seq_length()
        h = self.embed_tokens(input_ids)
        pos = self.rotary_emb.tokens(start, input_ids.shape[1])
        blk = self.rotary_emb.blocks()
        residual = None
        for layer in self.layers:
            h, residual = layer(h, pos, blk, past_key_values, residual)
        return self.norm(h, residual)[1]


class CompactAttnLlamaForCausalLM(nn.Module):
    """Decoder + LM head; forward(input_ids, past_key_values, logits_to_keep) runs one
    prefill chunk (the reference runtime's call, chunked_prefill_runtime.py:1168-1203) or,
    for a single token or once the cache length is inside a block, one dense decode step."""

    attn_cls: Type[nn.Module] = nn.Module
    cache_with_kmean = False
    cache_with_kgate = False

    def __init__(self, config: SeerAttnLlamaConfig, device=None):
        super().__init__()
        config.validate()
        self.config = config
        self.model = CompactAttnLlamaModel(config, self.attn_cls, device=device)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False, device=device, dtype=torch.bfloat16)

    @torch.no_grad()
    def init_weights(self, seed: int = 1234) -> None:
        """Random N(0, initializer_range) weights (unit RMSNorm weights), drawn on the
        parameters' device from one seeded generator."""
        dev = self.lm_head.weight.device
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        std = self.config.initializer_range
        for name, p in self.named_parameters():
            if name.endswith("layernorm.weight") or name == "model.norm.weight":
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=g)

    def new_cache(self, batch: int, max_tokens: int) -> ChunkedPrefillCache:
        return ChunkedPrefillCache(self.config, batch, max_tokens, self.lm_head.weight.device,
                                   with_kmean=self.cache_with_kmean, with_kgate=self.cache_with_kgate)

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, past_key_values: ChunkedPrefillCache,
                logits_to_keep: int = 1) -> torch.Tensor:
        h = self.model(input_ids, past_key_values)
        if logits_to_keep > 0:
            h = h[:, -logits_to_keep:]
        return self.lm_head(h)

    def attention_stats(self) -> List[Optional[dict]]:
        return [layer.self_attn._compactattn_last_stats for layer in self.model.layers]
