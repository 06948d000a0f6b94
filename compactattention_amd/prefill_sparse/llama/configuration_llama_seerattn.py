"""Configuration of the compactattn Llama models.

Field names follow the reference's SeerAttnLlamaConfig
(compact_attn/prefill_sparse/llama/configuration_llama_seerattn.py) and the config
attributes its compactattn modules read (modeling_llama_seerattn_chunked_dense.py:547-938,
modeling_llama_flashprefill_compactattn.py:60-120).  Defaults are the Llama-3.1-8B shape.
Only the fields this path uses are kept.  The Seer selector follows the reference's
compactattn layer: keep a past block when a query block's gate score exceeds
``seerattn_compactattn_threshold`` (looked up in ``seerattn_compactattn_threshold_schedule``
by the chunk's kv length when a schedule is given), plus the last
``seerattn_compactattn_keep_recent_blocks`` KV blocks; the current chunk is always kept.
The two ``compactattn_*_blocks`` fields add a sink / local-block rule that the reference does
not have (BASELINE configs 1 and 3 ask for it); they default to 0.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, fields
from typing import Any, Dict, Optional


@dataclass
class SeerAttnLlamaConfig:
    vocab_size: int = 128256
    hidden_size: int = 4096
    intermediate_size: int = 14336
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    max_position_embeddings: int = 131072
    initializer_range: float = 0.02
    # Seer AttnGate (attn_gate.py:37-278).  The defaults are the reference's
    # (configuration_llama_seerattn.py:191,198): Qavg_Kmaxminavg without force_double, i.e. no
    # query projection and W_k per Q head.  Every Q{pools}_K{pools} type with either setting
    # runs on the same kernels; BASELINE configs 1 and 3 use Qavg_Kavg with force_double
    # (compactattention_amd.synthetic.BASELINE_SEER).
    seerattn_gate_type: str = "Qavg_Kmaxminavg"
    seerattn_gate_block_size: int = 64
    seerattn_gate_hidden_size: int = 128
    seerattn_gate_force_double: bool = False
    seerattn_compactattn_kv_group_aware_gate: bool = False
    seerattn_sparsity_method: str = "threshold"
    seerattn_threshold: float = 0.0  # the block-sparse Seer layer's threshold (not read by this path)
    seerattn_chunked_prefill_force_dense: bool = False
    # the compactattn Seer layer's rule (modeling_llama_seerattn_chunked_dense.py:199-210,
    # configuration_llama_seerattn.py:199-200)
    seerattn_compactattn_threshold: float = 5e-4
    seerattn_compactattn_threshold_schedule: Optional[Any] = None
    seerattn_compactattn_keep_recent_blocks: int = 2
    compactattn_sink_blocks: int = 0
    compactattn_local_blocks: int = 0
    # FlashPrefill selector (modeling_llama_flashprefill_compactattn.py:253,266-293,486-491): score
    # blocks of 128 tokens by default as in the reference (64 or 128 here); BASELINE's FlashPrefill
    # configurations score 64-token blocks
    seerattn_flashprefill_block_size: int = 128
    seerattn_flashprefill_attention_sink: int = 2
    seerattn_flashprefill_window_size: int = 4
    seerattn_flashprefill_alpha: float = 0.06
    seerattn_flashprefill_last_n_block: int = 2
    seerattn_flashprefill_min_budget: int = 0
    # this build's choice of FlashPrefill score form: "pooled" (block means, bit-reproducible)
    # or "token" (the reference's per-token exp2 mass, compute_block_score_chunked)
    seerattn_flashprefill_score_mode: str = "pooled"

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> "SeerAttnLlamaConfig":
        names = {f.name for f in fields(cls)}
        unknown = set(d) - names
        if unknown:
            raise ValueError(f"unknown config fields: {sorted(unknown)}")
        return cls(**d)

    def to_dict(self) -> Dict[str, Any]:
        return asdict(self)

    @property
    def num_key_value_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    def validate(self) -> None:
        if self.head_dim != 128:
            raise ValueError("the compactattn kernels run head_dim 128")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        if self.seerattn_gate_block_size != 64:
            raise ValueError("the compactattn path runs 64-token blocks")
        if self.seerattn_flashprefill_block_size not in (64, 128):
            raise ValueError("FlashPrefill scoring runs 64- or 128-token blocks")
        if self.seerattn_flashprefill_score_mode not in ("pooled", "token"):
            raise ValueError("seerattn_flashprefill_score_mode must be 'pooled' or 'token'")
        from ..attn_gate import parse_gate_type

        parse_gate_type(self.seerattn_gate_type)
        if self.seerattn_gate_hidden_size != 128:
            raise ValueError("the gate kernels run a 128-dim gate hidden size")
        if self.seerattn_sparsity_method != "threshold":
            raise ValueError("the Seer selector implemented here is the softmax threshold")
