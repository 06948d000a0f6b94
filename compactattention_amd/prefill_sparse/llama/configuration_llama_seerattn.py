"""Configuration of the compactattn Llama models.

Field names follow the reference's SeerAttnLlamaConfig
(compact_attn/prefill_sparse/llama/configuration_llama_seerattn.py) and the config
attributes its compactattn modules read (modeling_llama_seerattn_chunked_dense.py:547-938,
modeling_llama_flashprefill_compactattn.py:60-120).  Defaults are the Llama-3.1-8B shape.
Only the fields this path uses are kept; the two `compactattn_*_blocks` fields are this
build's sink / local-block rule for the Seer selector (the reference keeps the current
chunk's blocks only).
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, fields
from typing import Any, Dict


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
    # Seer AttnGate (attn_gate.py:37-278).  The defaults are BASELINE config 1's gate (pooled
    # Q and K, both projected per head); the reference's own default is Qavg_Kmaxminavg
    # without force_double (configuration_llama_seerattn.py:191,198), and every
    # Q{pools}_K{pools} type with either setting runs on the same kernels.
    seerattn_gate_type: str = "Qavg_Kavg"
    seerattn_gate_block_size: int = 64
    seerattn_gate_hidden_size: int = 128
    seerattn_gate_force_double: bool = True
    seerattn_compactattn_kv_group_aware_gate: bool = False
    seerattn_sparsity_method: str = "threshold"
    seerattn_threshold: float = 5e-3
    seerattn_chunked_prefill_force_dense: bool = False
    seerattn_compactattn_keep_recent_blocks: int = 2
    compactattn_sink_blocks: int = 1
    compactattn_local_blocks: int = 2
    # FlashPrefill selector (modeling_llama_flashprefill_compactattn.py:266-293)
    seerattn_flashprefill_block_size: int = 64
    seerattn_flashprefill_attention_sink: int = 2
    seerattn_flashprefill_window_size: int = 4
    seerattn_flashprefill_alpha: float = 0.06
    seerattn_flashprefill_last_n_block: int = 2
    seerattn_flashprefill_min_budget: int = 0

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
        if self.seerattn_gate_block_size != 64 or self.seerattn_flashprefill_block_size != 64:
            raise ValueError("the compactattn path runs 64-token blocks")
        from ..attn_gate import parse_gate_type

        parse_gate_type(self.seerattn_gate_type)
        if self.seerattn_gate_hidden_size != 128:
            raise ValueError("the gate kernels run a 128-dim gate hidden size")
        if self.seerattn_sparsity_method != "threshold":
            raise ValueError("the Seer selector implemented here is the softmax threshold")
