"""Seer (AttnGate) compactattn Llama attention and model on the HIP kernels.

Mirrors LlamaSeerAttentionChunkedDense.forward
(compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:547-938):
q/k/v projections, RoPE, cache update, the gate K-block cache (:385-478), then for a
chunk with past context the compactattn forward (threshold on the AttnGate softmax scores,
Q-block union, GQA union, indexed attention), for the first chunk dense causal attention,
then o_proj.  The module returns the reference's 5-tuple (attn_output, mask_loss, None,
attn_gate_output, ground_truth_mask); inference only.

Execution per chunk (B requests advancing together, L tokens, P past blocks):
  1. paged append of RoPE'd K and V (ca_cache_fill, copy only);
  2. gate K summaries of the new blocks from the pre-RoPE K (ca_gate_key_summaries: the
     gate type's pools -> per-head projection -> block RoPE) into the cache's kgate;
  3. pooled (projected, rotated) query blocks (ca_gate_query_summaries);
  4. gate scores + per-row rule (ca_score_select: softmax over causal key blocks,
     keep score > threshold, the last keep_recent_blocks KV blocks; optional sink and local
     blocks, off by default);
  5. Q-block and GQA union into per-KV-group tables (ca_union_compact);
  6. indexed attention over the cache pages (ca_attn_fwd).
Steps 2-5 replace the reference's _compute_chunked_gate_from_cache + AttnGate +
chunked_prefill_column_dense_attention_forward; their bits are pinned by the kernel tests
against the CPU oracle.
"""
from __future__ import annotations

import json
import os
from typing import Any, Optional, Tuple

import torch
from torch import nn

from ... import ops
from ...modules._core import COMPACTATTN_VERSION
from ...modules.attention_forward_chunked_dense import (_compactattn_effective_threshold,
                                                        _compactattn_keep_recent_blocks, keep_recent_local_blocks)
from ..attn_gate import ATTNGATE_CLASSES
from .configuration_llama_seerattn import SeerAttnLlamaConfig
from .modeling_llama_common import (ChunkedPrefillCache, CompactAttnLlamaForCausalLM, FusedProjections,
                                     dense_decode_forward, event_span, is_decode_step, project_qkv, rope_qk)

BLOCK = 64


def normalize_compactattn_threshold_schedule(schedule: Optional[Any]) -> Optional[dict]:
    """A kv-length threshold schedule in the reference's forms
    (modeling_llama_seerattn_chunked_dense.py:36-84): None, a JSON file path, a list of entries
    or a dict with ``entries``; each entry {"max_kv_len": n > 0, "threshold": t}, t raised to the
    schedule's ``threshold_lower_bound`` (default 0.0).  Returns the dict with its entries sorted
    by max_kv_len."""
    if schedule is None:
        return None
    if isinstance(schedule, str):
        with open(os.path.expanduser(schedule), "r", encoding="utf-8") as f:
            schedule = json.load(f)
    if isinstance(schedule, (list, tuple)):
        schedule = {"entries": list(schedule)}
    if not isinstance(schedule, dict):
        raise TypeError("seerattn_compactattn_threshold_schedule must be None, a JSON path, a dict, or a list of "
                        f"entries; got {type(schedule)!r}")
    raw = schedule.get("entries")
    if raw is None:
        raise ValueError("Threshold schedule must contain an 'entries' field.")
    if not isinstance(raw, list) or not raw:
        raise ValueError("Threshold schedule 'entries' must be a non-empty list.")
    floor = float(schedule.get("threshold_lower_bound", 0.0))
    entries = []
    for i, e in enumerate(raw):
        if not isinstance(e, dict):
            raise TypeError(f"Schedule entry {i} must be a dict, got {type(e)!r}")
        if "max_kv_len" not in e or "threshold" not in e:
            raise ValueError(f"Schedule entry {i} must contain 'max_kv_len' and 'threshold'.")
        n = int(e["max_kv_len"])
        if n <= 0:
            raise ValueError(f"Schedule entry {i} has invalid max_kv_len={n}.")
        entries.append({"max_kv_len": n, "threshold": max(float(e["threshold"]), floor)})
    entries.sort(key=lambda e: e["max_kv_len"])
    return {**schedule, "entries": entries}


def resolve_compactattn_threshold(schedule: Optional[dict], kv_len: int, default_threshold: float) -> float:
    """The first entry (by max_kv_len) with kv_len <= max_kv_len, else the last entry; the
    default threshold without a schedule (reference :87-98)."""
    if not schedule:
        return float(default_threshold)
    for e in schedule["entries"]:
        if int(kv_len) <= e["max_kv_len"]:
            return float(e["threshold"])
    return float(schedule["entries"][-1]["threshold"])


class LlamaSeerAttentionChunkedDense(nn.Module):
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
        self.attn_gate = ATTNGATE_CLASSES[config.seerattn_gate_type](
            config.seerattn_gate_block_size, self.head_dim, config.seerattn_gate_hidden_size,
            num_k_head=self.num_key_value_heads, num_q_head=self.num_heads,
            force_double=config.seerattn_gate_force_double,
            kv_group_aware_query=config.seerattn_compactattn_kv_group_aware_gate).to(device)
        self.compactattn_threshold = float(config.seerattn_compactattn_threshold)
        self.compactattn_threshold_schedule = normalize_compactattn_threshold_schedule(
            config.seerattn_compactattn_threshold_schedule)
        self.compactattn_keep_recent_blocks = int(config.seerattn_compactattn_keep_recent_blocks)
        self.compactattn_version = COMPACTATTN_VERSION
        self.compactattn_debug = False
        self._compactattn_last_stats = None

    def _resolve_compactattn_threshold(self, kv_len: int) -> float:
        return resolve_compactattn_threshold(self.compactattn_threshold_schedule, kv_len, self.compactattn_threshold)

    def _selection_rule(self, q_blocks: int, kv_len: int) -> ops.Rule:
        """The reference layer's rule for a chunk of q_blocks query blocks ending at kv_len:
        the threshold from the schedule (debug override applied as in the operator entry), the
        last keep_recent_blocks KV blocks forced; plus this build's optional sink / local blocks."""
        c = self.config
        thr = _compactattn_effective_threshold(self._resolve_compactattn_threshold(kv_len))
        recent = keep_recent_local_blocks(_compactattn_keep_recent_blocks(self.compactattn_keep_recent_blocks),
                                          q_blocks)
        return ops.Rule(threshold=float(thr), sink_blocks=c.compactattn_sink_blocks,
                        local_blocks=max(int(c.compactattn_local_blocks), recent))

    def _append_compactattn_chunked_gate_key_cache(self, key_states_nope: torch.Tensor, cache, past: int,
                                                   block_position_embeddings) -> None:
        self.attn_gate.compress_key_blocks(key_states_nope, out=cache.kgate, first_block=past,
                                           position_embeddings=block_position_embeddings)
        if cache.kgate_blocks == past:  # a gap left by decode-completed blocks stays a gap
            cache.kgate_blocks = past - (-key_states_nope.shape[1] // BLOCK)  # a partial block's summary counts

    def _select_tables(self, query_states_nope: torch.Tensor, cache, past: int, block_position_embeddings
                       ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Gate scores per Q head (or per KV head for a kv-group-aware gate), threshold rule,
        then the Q-block and GQA unions into per-KV-group tables."""
        B = query_states_nope.shape[0]
        P = [past] * B
        gate = self.attn_gate
        qhat = gate.compress_query_blocks(query_states_nope, first_block=past,
                                          position_embeddings=block_position_embeddings, kv_cap=cache.cap)
        q_blocks = -(-query_states_nope.shape[1] // BLOCK)
        rule = self._selection_rule(q_blocks, 64 * past + query_states_nope.shape[1])
        rowmask, _ = ops.score_select(qhat, cache.kgate, gate.scale, rule, P, gate.key_heads, cache.cap)
        table, counts, _, _ = ops.union_compact(rowmask, P, self.num_key_value_heads, cache.cap)
        return table, counts

    def _do_chunked_compactattn_attention(self, query_states: torch.Tensor, query_states_nope: torch.Tensor, cache,
                                          past: int, block_position_embeddings, dense: bool):
        B, L = query_states.shape[:2]
        P = [past] * B
        if dense:
            table, counts = ops.dense_table(P, L, self.num_heads, self.num_key_value_heads, cache.cap,
                                            query_states.device)
        else:
            table, counts = self._select_tables(query_states_nope, cache, past, block_position_embeddings)
        K, V = cache.layouts()
        out = ops.attn_fwd(query_states, K, V, table, counts, P, self.scaling, cache.cap, self.num_key_value_heads)
        return out, table, counts

    def forward(self, hidden_states: torch.Tensor, position_embeddings: Tuple[torch.Tensor, torch.Tensor],
                attention_mask: Optional[torch.Tensor] = None, past_key_value: Optional[ChunkedPrefillCache] = None,
                cache_position: Optional[torch.LongTensor] = None,
                block_position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, **kwargs):
        del cache_position, kwargs
        if past_key_value is None:
            raise ValueError("the compactattn prefill path needs a ChunkedPrefillCache")
        if attention_mask is not None and not bool(attention_mask.all()):
            raise ValueError("padded positions are not supported by the compactattn prefill path")
        if block_position_embeddings is None:
            raise ValueError("block_position_embeddings (per-block rotary tables) are required")
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
            past = cache.append(key_states, v)  # v, k and q may be strided views of the fused GEMM
            self._append_compactattn_chunked_gate_key_cache(k, cache, past, block_position_embeddings)
            dense = past == 0 or bool(self.config.seerattn_chunked_prefill_force_dense)
            if not dense:
                cache.require_kgate(past)
            out, table, counts = self._do_chunked_compactattn_attention(query_states, q, cache, past,
                                                                       block_position_embeddings, dense)
        if self.table_sink is not None:  # per-chunk block counts (device tensors), for FLOP accounting
            self.table_sink.append((counts, L, past))
        out = self.o_proj(out.reshape(B, L, -1))
        if self.compactattn_debug:
            self._compactattn_last_stats = {
                "path": "first_chunk_dense" if past == 0 else ("forced_dense" if dense else "chunked_selected"),
                "past_blocks": past, "table": table, "counts": counts,
                "compactattn_version": self.compactattn_version,
            }
        else:
            self._compactattn_last_stats = None
        return out, 0.0, None, None, None


class SeerAttnLlamaChunkedDenseForCausalLM(CompactAttnLlamaForCausalLM):
    attn_cls = LlamaSeerAttentionChunkedDense
    cache_with_kgate = True
