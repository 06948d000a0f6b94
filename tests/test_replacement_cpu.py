"""The stock-transformers attention replacement (load_attention_replacement) on the CPU:
structure, shared projections, parameter names, gate-weight loading and argument errors.
The GPU test of its outputs is tests/test_gpu_model.py::test_hf_replacement_*."""
from __future__ import annotations

import os

import pytest
import torch

transformers = pytest.importorskip("transformers")

from compactattention_amd.load_attention_replacement import (  # noqa: E402
    load_llama_attention_replacement_model, new_compactattn_cache)
from compactattention_amd.prefill_sparse.llama import (  # noqa: E402
    LlamaFlashPrefillCompactAttnAttention, LlamaSeerAttentionChunkedDense)


def _stock(layers=2):
    cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                                   max_position_embeddings=2048)
    torch.manual_seed(0)
    return transformers.LlamaForCausalLM(cfg)


@pytest.mark.parametrize("variant,cls", [("seer_compactattn", LlamaSeerAttentionChunkedDense),
                                         ("seer_compactattn_hf", LlamaSeerAttentionChunkedDense),
                                         ("flashprefill_compactattn", LlamaFlashPrefillCompactAttnAttention)])
def test_replacement_structure(variant, cls):
    m = _stock()
    projs = [(l.self_attn.q_proj, l.self_attn.o_proj) for l in m.model.layers]
    r = load_llama_attention_replacement_model(base_model=m, variant=variant, threshold=1e-3)
    assert r.config._attn_implementation == "compactattn"
    assert r.config.seerattn_attention_harness == "replacement"
    for layer, (q, o) in zip(r.model.layers, projs):
        assert isinstance(layer.self_attn, cls)
        assert layer.self_attn.q_proj is q and layer.self_attn.o_proj is o
    keys = [k for k in r.state_dict() if k.startswith("model.layers.0.self_attn.")]
    if variant.startswith("seer"):
        # the reference's default gate (Qavg_Kmaxminavg, no force_double): no query
        # projection, W_k per Q head over the 3 x 128 pooled K inputs
        gate = r.model.layers[0].self_attn.attn_gate
        assert gate.mask_linear_q is None
        assert "model.layers.0.self_attn.attn_gate.mask_linear_k.weight" in keys
        assert tuple(gate.mask_linear_k.weight.shape) == (4, 384, 128)
        assert gate.mask_linear_k.weight.dtype == torch.float32
    cache = new_compactattn_cache(r, 1, 256)
    assert cache.layer(0).kgate is not None if variant.startswith("seer") else cache.layer(0).kmean is not None
    # the HIP path has no CPU fallback
    with pytest.raises(ValueError, match="GPU tensor"):
        r(input_ids=torch.randint(0, 512, (1, 128)), past_key_values=cache, use_cache=True, logits_to_keep=1)


def test_replacement_argument_errors(tmp_path):
    with pytest.raises(ValueError, match="unsupported variant"):
        load_llama_attention_replacement_model(base_model=_stock(), variant="seer_block_sparse")
    with pytest.raises(ValueError, match="64- or 128-token blocks"):
        load_llama_attention_replacement_model(base_model=_stock(), variant="flashprefill_compactattn",
                                               flashprefill_block_size=256)
    # the reference's default FlashPrefill block (128 tokens) is the loader's default
    fp = load_llama_attention_replacement_model(base_model=_stock(), variant="flashprefill_compactattn")
    assert fp.compactattn_config.seerattn_flashprefill_block_size == 128
    r = load_llama_attention_replacement_model(base_model=_stock(), variant="seer_compactattn")
    with pytest.raises(ValueError, match="past_key_values"):
        r(input_ids=torch.randint(0, 512, (1, 64)), use_cache=False)
    with pytest.raises(ValueError, match="not found"):
        load_llama_attention_replacement_model(base_model=_stock(), variant="seer_compactattn",
                                               model_id=str(tmp_path / "missing"))


def test_gate_weights_load_by_reference_key_names(tmp_path):
    ref = load_llama_attention_replacement_model(base_model=_stock(), variant="seer_compactattn")
    state = {k: torch.randn_like(v) for k, v in ref.state_dict().items() if ".attn_gate." in k}
    torch.save(state, os.path.join(tmp_path, "attn_gate_weights.pth"))
    r = load_llama_attention_replacement_model(base_model=_stock(), variant="seer_compactattn", model_id=str(tmp_path))
    got = r.state_dict()
    for k, v in state.items():
        assert torch.equal(got[k], v)
    torch.save({"model.layers.0.self_attn.attn_gate.nope": torch.zeros(1)}, os.path.join(tmp_path, "bad.pth"))
    with pytest.raises(ValueError, match="not in the model"):
        load_llama_attention_replacement_model(base_model=_stock(), variant="seer_compactattn",
                                               model_id=os.path.join(tmp_path, "bad.pth"))


def test_gate_settings_from_checkpoint_config(tmp_path):
    """The gate type, force_double and the kv-group-aware flag come from the gate checkpoint's
    config.json, as the reference reads them with SeerAttnLlamaConfig.from_pretrained(model_id)."""
    import json

    # a Qavg_Kavg / force_double checkpoint: both projections per head, loaded by the
    # reference's key names
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump({"seerattn_gate_type": "Qavg_Kavg", "seerattn_gate_force_double": True}, f)
    gate_state = {}
    for i in range(2):
        gate_state[f"model.layers.{i}.self_attn.attn_gate.mask_linear_q.weight"] = torch.randn(4, 128, 128)
        gate_state[f"model.layers.{i}.self_attn.attn_gate.mask_linear_k.weight"] = torch.randn(2, 128, 128)
    torch.save(gate_state, os.path.join(tmp_path, "attn_gate_weights.pth"))
    r = load_llama_attention_replacement_model(base_model=_stock(), variant="seer_compactattn", model_id=str(tmp_path))
    assert r.compactattn_config.seerattn_gate_type == "Qavg_Kavg" and r.compactattn_config.seerattn_gate_force_double
    got = r.state_dict()
    for k, v in gate_state.items():
        assert torch.equal(got[k], v)
    cache = new_compactattn_cache(r, 1, 256)
    assert cache.layer(0).kgate.shape[1] == 2  # gate K per KV head
    # kv-group-aware gate (the other settings at the reference's defaults): W_q [Hkv, G*128, 128],
    # scores per KV head
    kv_dir = tmp_path / "kv"
    os.makedirs(kv_dir)
    with open(os.path.join(kv_dir, "config.json"), "w") as f:
        json.dump({"seerattn_compactattn_kv_group_aware_gate": True}, f)
    torch.save({}, os.path.join(kv_dir, "attn_gate_weights.pth"))
    r = load_llama_attention_replacement_model(base_model=_stock(), variant="seer_compactattn", model_id=str(kv_dir))
    gate = r.model.layers[0].self_attn.attn_gate
    assert gate.kv_group_aware_query and tuple(gate.mask_linear_q.weight.shape) == (2, 2 * 128, 128)
    assert gate.query_heads == 2 and gate.key_heads == 2
