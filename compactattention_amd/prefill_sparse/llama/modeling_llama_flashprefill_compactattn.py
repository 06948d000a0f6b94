"""FlashPrefill compactattn Llama attention and model on the HIP kernels.

Mirrors LlamaFlashPrefillCompactAttnAttention.forward
(compact_attn/prefill_sparse/llama/modeling_llama_flashprefill_compactattn.py:152-341):
q/k/v projections, RoPE, cache update with the per-layer mean-K cache (:121-150), then
flashprefill_compactattn_prefill_full_kv for chunks with past context and dense attention
for the first chunk, then o_proj.

Execution per chunk: one ca_cache_fill_pool_query launch appends the RoPE'd K/V pages,
writes the fp32 mean-K of the new blocks and pools the RoPE'd queries (a first or forced-dense
chunk only appends, through ca_cache_fill); ca_score_select scores
pooled Q.K blocks (softmax over causal key blocks, scale 1/sqrt(128)) and applies the
FlashPrefill row rule (alpha * row max, sink, window, optional top-k budget);
ca_union_compact leaves the last last_n_block query blocks out of the union; ca_attn_fwd
attends over the cache pages.  With seerattn_flashprefill_block_size 128 (the reference's
default) the pooled query and key means are paired into 128-token blocks
(ca_pair_block_summaries) before scoring, and the tables name both 64-token pages of each
selected block.  A chunk that is not a multiple of 64 tokens selects with a partial last
block.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import nn

from ... import ops
from ...modules._core import COMPACTATTN_VERSION
from ...modules.flashprefill_prefill import flashprefill_rule, flashprefill_tables
from .configuration_llama_seerattn import SeerAttnLlamaConfig
from .modeling_llama_common import (ChunkedPrefillCache, CompactAttnLlamaForCausalLM, FusedProjections,
                                     dense_decode_forward, event_span, is_decode_step, project_qkv, rope_qk)

BLOCK = 64


class LlamaFlashPrefillCompactAttnAttention(nn.Module):
    def __init__(self, config: SeerAttnLlamaConfig, layer_idx: int, device=None):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = config.head_dim
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_key_value_groups = config.num_key_value_groups
        self.scaling = self.head_dim ** -0.5
        kw = dict(bias=False, device=device, dtype=torch.bfloat16)
        self.q_proj = nn.Linear(config.hidden_size, self.num_heads * self.head_dim, **kw)
        self.k_proj = nn.Linear(config.hidden_size, self.num_key_value_heads * self.head_dim, **kw)
        self.v_proj = nn.Linear(config.hidden_size, self.num_key_value_heads * self.head_dim, **kw)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, config.hidden_size, **kw)
        self.qkv = FusedProjections(self, ("q_proj", "k_proj", "v_proj"))
        self.attention_timer: Optional[list] = None  # a list collects timing events of the attention core
        self.table_sink: Optional[list] = None  # a list collects (counts, chunk length, past blocks) per call
        self.compactattn_version = COMPACTATTN_VERSION
        self.compactattn_debug = False
        self._compactattn_last_stats = None

    def _selection_rule(self) -> ops.Rule:
        c = self.config
        return flashprefill_rule(c.seerattn_flashprefill_attention_sink, c.seerattn_flashprefill_window_size,
                                 c.seerattn_flashprefill_alpha, c.seerattn_flashprefill_last_n_block,
                                 c.seerattn_flashprefill_min_budget)

    def forward(self, hidden_states: torch.Tensor, position_embeddings: Tuple[torch.Tensor, torch.Tensor],
                attention_mask: Optional[torch.Tensor] = None, past_key_value: Optional[ChunkedPrefillCache] = None,
                cache_position: Optional[torch.LongTensor] = None, **kwargs):
        del cache_position, kwargs
        if past_key_value is None:
            raise ValueError("the compactattn prefill path needs a ChunkedPrefillCache")
        if attention_mask is not None and not bool(attention_mask.all()):
            raise ValueError("padded positions are not supported by the compactattn prefill path")
        if is_decode_step(hidden_states, past_key_value.layer(self.layer_idx)):
            out = dense_decode_forward(self, hidden_states, position_embeddings, past_key_value.layer(self.layer_idx))
            self._compactattn_last_stats = {"path": "decode_dense"} if self.compactattn_debug else None
            return out, 0.0, None, None, None
        B, L, _ = hidden_states.shape
        q, k, v = project_qkv(self, hidden_states)
        cos, sin = position_embeddings
        with event_span(self.attention_timer):
            query_states, key_states = rope_qk(q, k, cos, sin)
            cache = past_key_value.layer(self.layer_idx)
            dense = cache.past_blocks == 0 or bool(self.config.seerattn_chunked_prefill_force_dense)
            if dense:
                past = cache.append(key_states, v)  # pages + mean-K of the new blocks (v may be strided)
            else:  # the same append and the pooled queries in one launch
                past, qhat = cache.append_with_query_means(key_states, v, query_states)
            P = [past] * B
            if dense:
                table, counts = ops.dense_table(P, L, self.num_heads, self.num_key_value_heads, cache.cap,
                                                query_states.device)
            else:  # score blocks of seerattn_flashprefill_block_size (64 or 128) tokens
                table, counts = flashprefill_tables(qhat, cache.kmean, P, L, self.num_key_value_heads, cache.cap,
                                                    self._selection_rule(),
                                                    self.config.seerattn_flashprefill_block_size,
                                                    score_mode=self.config.seerattn_flashprefill_score_mode,
                                                    query_states=query_states)
            K, V = cache.layouts()
            out = ops.attn_fwd(query_states, K, V, table, counts, P, self.scaling, cache.cap,
                               self.num_key_value_heads)
        if self.table_sink is not None:  # per-chunk block counts (device tensors), for FLOP accounting
            self.table_sink.append((counts, L, past))
        out = self.o_proj(out.reshape(B, L, -1))
        if self.compactattn_debug:
            self._compactattn_last_stats = {
                "path": "dense_fallback" if dense else "flashprefill_chunked_selected",
                "past_blocks": past, "table": table, "counts": counts,
                "compactattn_version": self.compactattn_version,
            }
        else:
            self._compactattn_last_stats = None
        return out, 0.0, None, None, None


class SeerAttnLlamaFlashPrefillCompactAttnForCausalLM(CompactAttnLlamaForCausalLM):
    attn_cls = LlamaFlashPrefillCompactAttnAttention
    cache_with_kmean = True
