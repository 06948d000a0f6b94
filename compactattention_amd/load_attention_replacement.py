"""Stock Hugging Face Llama with its attention modules replaced by the compactattn ones.

Mirrors load_llama_attention_replacement_model
(compact_attn/load_attention_replacement.py:236-336): the decoder layers, norms, MLPs and
rotary embedding stay the transformers implementation, and each layer's ``self_attn`` becomes
the Seer or FlashPrefill compactattn module of this package.  The replacement reuses the stock
q/k/v/o projection modules, keeps its parameters under ``self_attn.*`` (so gate weights load
by the reference's key names) and returns the transformers 2-tuple ``(attn_output, None)``.

Differences from the reference, each raised as ``ValueError`` rather than ignored:
- only the compactattn variants (``seer_compactattn``, ``seer_compactattn_hf``,
  ``flashprefill_compactattn``) exist here; the block-sparse variants are outside this path;
- ``base_model`` is a transformers ``LlamaForCausalLM`` instance or a local directory (there
  is no hub download), and gate weights load from a local ``attn_gate_weights.pth`` with
  ``torch.load(weights_only=True)``.

The KV cache is this package's paged cache: pass ``past_key_values=new_compactattn_cache(...)``
to the model (transformers' DynamicCache is not read).  The model's attention implementation
is set to ``"compactattn"``, which has no mask function, so transformers builds no dense
causal mask; the compactattn modules apply causality themselves.
"""
from __future__ import annotations

import os
from types import MethodType
from typing import Optional, Union

import torch
from torch import nn

from .prefill_sparse.llama.configuration_llama_seerattn import SeerAttnLlamaConfig
from .prefill_sparse.llama.modeling_llama_common import ChunkedPrefillCache
from .prefill_sparse.llama.modeling_llama_flashprefill_compactattn import LlamaFlashPrefillCompactAttnAttention
from .prefill_sparse.llama.modeling_llama_seerattn_chunked_dense import LlamaSeerAttentionChunkedDense

BLOCK = 64
ATTN_IMPLEMENTATION = "compactattn"
_VARIANTS = {
    "seer_compactattn": LlamaSeerAttentionChunkedDense,
    "seer_compactattn_hf": LlamaSeerAttentionChunkedDense,
    "flashprefill_compactattn": LlamaFlashPrefillCompactAttnAttention,
}


def _register_attention_implementation() -> None:
    """A named attention implementation without a mask function: transformers' mask builder
    returns None for it (masking_utils._preprocess_mask_arguments exits early)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS, AttentionInterface

    if ATTN_IMPLEMENTATION in ALL_ATTENTION_FUNCTIONS._global_mapping:
        return

    def _unused(*args, **kwargs):
        raise RuntimeError("the compactattn modules replace the attention call itself")

    AttentionInterface.register(ATTN_IMPLEMENTATION, _unused)


def _rope_theta(hf_config) -> float:
    theta = getattr(hf_config, "rope_theta", None)
    if theta is None:
        params = getattr(hf_config, "rope_parameters", None) or {}
        theta = params.get("rope_theta", 10000.0)
    return float(theta)


# The gate settings of the reference's SeerAttnLlamaConfig defaults
# (compact_attn/prefill_sparse/llama/configuration_llama_seerattn.py:191,198,202), which apply
# when the gate checkpoint's config.json does not set them.
_GATE_DEFAULTS = {
    "seerattn_gate_type": "Qavg_Kmaxminavg",
    "seerattn_gate_force_double": False,
    "seerattn_compactattn_kv_group_aware_gate": False,
}


def _gate_settings(model_id: Optional[str]) -> dict:
    """Gate type / force_double / kv-group-aware flag from the gate checkpoint's config.json
    (a local directory; plain JSON), else the reference's defaults -- the reference reads the
    same fields through SeerAttnLlamaConfig.from_pretrained(model_id)
    (compact_attn/load_attention_replacement.py:131-132)."""
    import json

    out = dict(_GATE_DEFAULTS)
    if model_id is None or not os.path.isdir(model_id):
        return out
    path = os.path.join(model_id, "config.json")
    if os.path.isfile(path):
        with open(path) as f:
            cfg = json.load(f)
        for key in out:
            if key in cfg:
                out[key] = type(_GATE_DEFAULTS[key])(cfg[key])
    return out


def _build_seer_config(hf_config, *, variant: str, threshold: float, compactattn_keep_recent_blocks: int,
                       flashprefill_alpha: float, flashprefill_block_size: int, flashprefill_attention_sink: int,
                       flashprefill_window_size: int, flashprefill_last_n_block: int,
                       flashprefill_min_budget: int, gate: Optional[dict] = None) -> SeerAttnLlamaConfig:
    head_dim = getattr(hf_config, "head_dim", None) or hf_config.hidden_size // hf_config.num_attention_heads
    cfg = SeerAttnLlamaConfig(
        vocab_size=hf_config.vocab_size,
        hidden_size=hf_config.hidden_size,
        intermediate_size=hf_config.intermediate_size,
        num_hidden_layers=hf_config.num_hidden_layers,
        num_attention_heads=hf_config.num_attention_heads,
        num_key_value_heads=getattr(hf_config, "num_key_value_heads", None) or hf_config.num_attention_heads,
        head_dim=head_dim,
        rms_norm_eps=float(hf_config.rms_norm_eps),
        rope_theta=_rope_theta(hf_config),
        max_position_embeddings=hf_config.max_position_embeddings,
        # the reference sets both thresholds and no schedule (load_attention_replacement.py:136-144);
        # no sink or local blocks: the Seer layer keeps the last keep_recent_blocks KV blocks
        seerattn_threshold=float(threshold),
        seerattn_compactattn_threshold=float(threshold),
        seerattn_compactattn_threshold_schedule=None,
        seerattn_compactattn_keep_recent_blocks=int(compactattn_keep_recent_blocks),
        seerattn_flashprefill_alpha=float(flashprefill_alpha),
        seerattn_flashprefill_block_size=int(flashprefill_block_size),
        seerattn_flashprefill_attention_sink=int(flashprefill_attention_sink),
        seerattn_flashprefill_window_size=int(flashprefill_window_size),
        seerattn_flashprefill_last_n_block=int(flashprefill_last_n_block),
        seerattn_flashprefill_min_budget=int(flashprefill_min_budget),
        **(gate or {}),
    )
    cfg.validate()
    return cfg


class _BlockRope:
    """Per-block rotary tables (positions 0, 64, 128, ...) from the stock rotary module, fp32,
    built once per device: the Seer gate rotates its pooled K/Q at each block's first position
    (the reference's ``model.model.block_rotary_emb``)."""

    def __init__(self, rotary: nn.Module, max_positions: int):
        self.rotary = rotary
        self.max_positions = max_positions
        self.tables = {}

    def get(self, device) -> tuple:
        key = str(device)
        if key not in self.tables:
            pos = torch.arange(0, self.max_positions, BLOCK, device=device)[None]
            x = torch.zeros((1, 1, 1), dtype=torch.float32, device=device)
            cos, sin = self.rotary(x, position_ids=pos)
            self.tables[key] = (cos[0].float().contiguous(), sin[0].float().contiguous())
        return self.tables[key]


def _adapt_to_transformers(attn: nn.Module, block_rope: _BlockRope) -> None:
    """transformers calls self_attn(hidden_states=..., attention_mask=..., position_ids=...,
    past_key_values=..., use_cache=..., position_embeddings=(cos, sin) [B, L, D]) and unpacks
    (attn_output, attn_weights)."""
    original = attn.forward

    def _forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_values=None, use_cache=None,
                 position_embeddings=None, **kwargs):
        del position_ids, use_cache, kwargs
        if not isinstance(past_key_values, ChunkedPrefillCache):
            raise ValueError("pass past_key_values=new_compactattn_cache(model, batch, max_tokens): the compactattn "
                             "modules keep their KV in the paged cache")
        if position_embeddings is None:
            raise ValueError("position_embeddings are required")
        cos, sin = position_embeddings
        if cos.dim() == 3:
            if cos.shape[0] > 1 and not torch.equal(cos[0], cos[-1]):
                raise ValueError("every request of a batch must sit at the same positions")
            cos, sin = cos[0], sin[0]
        out = original(hidden_states, (cos.float(), sin.float()), attention_mask, past_key_value=past_key_values,
                       block_position_embeddings=block_rope.get(hidden_states.device))
        return out[0], None

    attn.forward = MethodType(_forward, attn)


def _load_gate_weights(model: nn.Module, model_id: str) -> None:
    path = os.path.join(model_id, "attn_gate_weights.pth") if os.path.isdir(model_id) else model_id
    if not os.path.isfile(path):
        raise ValueError(f"gate weights not found at {path} (local files only; there is no hub download)")
    state = torch.load(path, map_location="cpu", weights_only=True)
    missing, unexpected = model.load_state_dict(state, strict=False)
    del missing
    if unexpected:
        raise ValueError(f"gate weight keys not in the model: {sorted(unexpected)[:4]} ...")


def load_llama_attention_replacement_model(
    *,
    base_model: Union[str, nn.Module],
    variant: str,
    model_id: Optional[str] = None,
    torch_dtype: torch.dtype = torch.bfloat16,
    device_map=None,
    threshold: float = 3e-4,
    compactattn_keep_recent_blocks: int = 2,
    flashprefill_alpha: float = 0.01,
    flashprefill_block_size: int = 128,
    flashprefill_attention_sink: int = 2,
    flashprefill_window_size: int = 4,
    flashprefill_last_n_block: int = 2,
    flashprefill_min_budget: int = 0,
) -> nn.Module:
    """Returns the stock LlamaForCausalLM with compactattn attention in every layer.

    base_model: a transformers LlamaForCausalLM (moved to torch_dtype) or a local model
    directory (``from_pretrained(..., local_files_only=True)``).  model_id: optional local
    directory or file holding the Seer gate weights (``attn_gate_weights.pth``).
    """
    from transformers import LlamaForCausalLM

    if variant not in _VARIANTS:
        raise ValueError(f"unsupported variant {variant!r}: this build has {sorted(_VARIANTS)}")
    if isinstance(base_model, nn.Module):
        model = base_model.to(dtype=torch_dtype)
    else:
        model = LlamaForCausalLM.from_pretrained(base_model, torch_dtype=torch_dtype, device_map=device_map,
                                                 local_files_only=True)
    model.eval()
    seer_cfg = _build_seer_config(
        model.config, variant=variant, threshold=threshold,
        compactattn_keep_recent_blocks=compactattn_keep_recent_blocks, flashprefill_alpha=flashprefill_alpha,
        flashprefill_block_size=flashprefill_block_size, flashprefill_attention_sink=flashprefill_attention_sink,
        flashprefill_window_size=flashprefill_window_size, flashprefill_last_n_block=flashprefill_last_n_block,
        flashprefill_min_budget=flashprefill_min_budget, gate=_gate_settings(model_id))
    block_rope = _BlockRope(model.model.rotary_emb, seer_cfg.max_position_embeddings)
    cls = _VARIANTS[variant]
    for layer_idx, layer in enumerate(model.model.layers):
        src = layer.self_attn
        dev = src.q_proj.weight.device
        impl = cls(seer_cfg, layer_idx, device=dev)
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(impl, name, getattr(src, name))
        impl.to(device=dev)  # the gate stays fp32, the projections keep the model's dtype
        impl.qkv.refuse()  # one GEMM for the stock q/k/v projections (weights re-seated, not copied)
        _adapt_to_transformers(impl, block_rope)
        layer.self_attn = impl
    model.eval()
    if variant != "flashprefill_compactattn" and model_id is not None:
        _load_gate_weights(model, model_id)
    _register_attention_implementation()
    model.config._attn_implementation = ATTN_IMPLEMENTATION
    model.config.seerattn_attention_harness = "replacement"
    model.config.seerattn_replacement_variant = variant
    model.config.seerattn_cache_layout = (
        "heads_first_flashprefill" if variant == "flashprefill_compactattn" else "heads_first_seer")
    model.compactattn_config = seer_cfg
    model.compactattn_block_rope = block_rope
    return model


def new_compactattn_cache(model: nn.Module, batch: int, max_tokens: int) -> ChunkedPrefillCache:
    """The paged cache the replaced attention modules read and append to."""
    cfg = getattr(model, "compactattn_config", None)
    if cfg is None:
        raise ValueError("not a compactattn replacement model")
    variant = model.config.seerattn_replacement_variant
    dev = model.model.embed_tokens.weight.device
    return ChunkedPrefillCache(cfg, batch, max_tokens, dev, with_kmean=variant == "flashprefill_compactattn",
                               with_kgate=variant != "flashprefill_compactattn")
