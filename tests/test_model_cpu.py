"""CPU checks of the compactattn model integration: configuration, construction, seeded
initialisation and argument errors (no kernel runs without a GPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from compactattention_amd.chunked_prefill import synthetic_prompt
from compactattention_amd.prefill_sparse.llama import (SeerAttnLlamaChunkedDenseForCausalLM, SeerAttnLlamaConfig,
                                                       SeerAttnLlamaFlashPrefillCompactAttnForCausalLM)
from compactattention_amd.prefill_sparse.llama.modeling_llama_common import apply_rotary_pos_emb, rotate_half


def tiny(**kw):
    base = dict(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=2,
                num_key_value_heads=1, max_position_embeddings=512)
    base.update(kw)
    return SeerAttnLlamaConfig(**base)


def test_default_config_is_llama_8b_shape():
    c = SeerAttnLlamaConfig()
    assert (c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads) == (4096, 32, 32, 8)
    assert (c.intermediate_size, c.vocab_size, c.rope_theta) == (14336, 128256, 500000.0)
    assert c.num_key_value_groups == 4
    c.validate()


def test_config_validation():
    with pytest.raises(ValueError, match="unknown config fields"):
        SeerAttnLlamaConfig.from_dict({"hidden_size": 8, "nope": 1})
    with pytest.raises(ValueError, match="64-token blocks"):
        tiny(seerattn_gate_block_size=128).validate()
    with pytest.raises(ValueError, match="head_dim 128"):
        tiny(head_dim=64).validate()
    # every gate type of the reference validates; malformed names do not
    tiny(seerattn_gate_type="Qmax_Kmax").validate()
    tiny(seerattn_gate_type="Qavg_Kmaxminavg", seerattn_gate_force_double=False).validate()
    with pytest.raises(ValueError, match="Q<pools>_K<pools>"):
        tiny(seerattn_gate_type="avg").validate()
    with pytest.raises(ValueError, match="unknown pooling name"):
        tiny(seerattn_gate_type="Qavg_Kmedian").validate()
    assert SeerAttnLlamaConfig.from_dict(tiny().to_dict()) == tiny()


@pytest.mark.parametrize("cls", [SeerAttnLlamaChunkedDenseForCausalLM, SeerAttnLlamaFlashPrefillCompactAttnForCausalLM])
def test_construction_and_seeded_init(cls):
    a = cls(tiny())
    b = cls(tiny())
    a.init_weights(seed=5)
    b.init_weights(seed=5)
    for (na, pa), (nb, pb) in zip(a.named_parameters(), b.named_parameters()):
        assert na == nb and torch.equal(pa, pb)
    assert torch.all(a.model.norm.weight == 1)
    assert a.lm_head.weight.dtype == torch.bfloat16
    names = {n for n, _ in a.named_parameters()}
    assert "model.layers.0.self_attn.q_proj.weight" in names
    if cls is SeerAttnLlamaChunkedDenseForCausalLM:
        # the reference's default gate: no query projection, W_k per Q head over max/min/avg K
        gate = a.model.layers[0].self_attn.attn_gate
        assert gate.mask_linear_q is None and gate.mask_linear_k.weight.shape == (2, 384, 128)
        b2 = cls(tiny(seerattn_gate_type="Qavg_Kavg", seerattn_gate_force_double=True))
        assert b2.model.layers[0].self_attn.attn_gate.mask_linear_q.weight.shape == (2, 128, 128)


def test_rope_matches_rotate_half_formula():
    g = torch.Generator().manual_seed(0)
    q = torch.randn((1, 8, 2, 128), generator=g)
    k = torch.randn((1, 8, 1, 128), generator=g)
    m = SeerAttnLlamaChunkedDenseForCausalLM(tiny())
    cos, sin = m.model.rotary_emb.tokens(3, 8)
    qr, kr = apply_rotary_pos_emb(q, k, cos, sin)
    # the rotation keeps each (i, i + 64) pair's norm and is the identity at position 0
    pair = lambda x: x[..., :64] ** 2 + x[..., 64:] ** 2  # noqa: E731
    assert torch.allclose(pair(qr), pair(q), atol=1e-5)
    c0, s0 = m.model.rotary_emb.tokens(0, 1)
    assert torch.allclose(apply_rotary_pos_emb(q[:, :1], k[:, :1], c0, s0)[0], q[:, :1])
    assert torch.equal(rotate_half(rotate_half(q)), -q)
    bc, bs = m.model.rotary_emb.blocks()
    assert torch.equal(bc[2], m.model.rotary_emb.cos[128])


def test_forward_rejects_cpu_tensors_for_prefill_and_decode():
    """The HIP path has no CPU fallback: a CPU model fails loudly in both prefill chunks and
    decode steps."""
    m = SeerAttnLlamaChunkedDenseForCausalLM(tiny())
    ids = synthetic_prompt(1, 128, 64, 0, "cpu")
    cache = m.new_cache(1, 192)
    with pytest.raises(ValueError, match="GPU tensor"):
        m(ids, cache)
    cache = m.new_cache(1, 192)
    with pytest.raises(ValueError, match="GPU tensor"):
        m(ids[:, :1], cache)


def test_paged_cache_decode_append_rules():
    from compactattention_amd.kv_cache import PagedKVCache

    c = PagedKVCache(1, 2, 192, "cpu")
    k = torch.randn((1, 67, 2, 128)).to(torch.bfloat16)
    v = torch.randn((1, 67, 2, 128)).to(torch.bfloat16)
    assert c.append_tokens(k[:, :64], v[:, :64]) == 0
    start = c.append_tokens(k[:, 64:], v[:, 64:])
    assert start == 64 and c.length == 67
    assert torch.equal(c.k_hf()[0], k[0].transpose(0, 1))
    assert torch.equal(c.v_hf()[0], v[0].transpose(0, 1))
    with pytest.raises(ValueError, match="partial block"):
        c.append(k[:, :64], k[:, :64])


def test_paged_cache_allocator_growth_fork_and_copy_on_write():
    """Host logic of the page pool and page table (CPU tensors; the kernels only read them):
    pages are handed out per (row, block) as the sequence grows, the pool and the page
    table grow past their initial size without moving any stored token, forked requests
    share pages by reference count, and a decode append into a shared partial page copies
    it first."""
    from compactattention_amd.kv_cache import PagedKVCache

    g = torch.Generator().manual_seed(0)
    c = PagedKVCache(2, 2, 128, "cpu", pool_pages=3)  # table for 2 blocks, 3 pages for 4 rows
    rows = 4
    toks = []
    for n in (64, 64, 40, 1):  # grows through 2 -> 4 blocks of table and 3 -> 16 pages
        k = torch.randn((2, n, 2, 128), generator=g).to(torch.bfloat16)
        c.append_tokens(k, -k)
        toks.append(k)
    allk = torch.cat(toks, dim=1)
    assert c.length == 169 and c.cap >= 3 and c.pool.num_pages >= rows * 3
    assert torch.equal(c.k_hf(), allk.transpose(1, 2)) and torch.equal(c.v_hf(), -allk.transpose(1, 2))
    # one distinct page per (row, block), the device table mirrors the host table
    pt = c.page_table.numpy()
    mapped = pt[:, :3]
    assert (mapped >= 0).all() and len(set(mapped.ravel().tolist())) == rows * 3
    assert (pt[:, 3:] == -1).all()
    assert (c.pool.refs[mapped.ravel()] == 1).all()
    # request 1 takes request 0's contents by sharing its pages
    free_before = c.pool.free_pages
    c.fork(0, 1)
    assert c.pool.free_pages == free_before + 2 * 3  # request 1's own pages came back
    assert np.array_equal(c.page_table.numpy()[2:4, :3], c.page_table.numpy()[0:2, :3])
    assert (c.pool.refs[c.page_table.numpy()[0:2, :3].ravel()] == 2).all()
    assert torch.equal(c.k_hf()[1], c.k_hf()[0])
    # decode append into the shared partial block 2: copy-on-write for both requests' rows
    k = torch.randn((2, 3, 2, 128), generator=g).to(torch.bfloat16)
    shared_page = int(c.page_table[0, 2])
    c.append_tokens(k, k)
    pt = c.page_table.numpy()
    assert pt[0, 2] != pt[2, 2] and shared_page in (pt[0, 2], pt[2, 2])
    assert np.array_equal(pt[0:2, :2], pt[2:4, :2])  # full blocks stay shared
    kk = c.k_hf()
    assert torch.equal(kk[0, :, :169], allk[0].transpose(0, 1))
    assert torch.equal(kk[1, :, :169], allk[0].transpose(0, 1))
    assert torch.equal(kk[:, :, 169:], k.transpose(1, 2))
    c.reset()
    assert c.length == 0 and c.pool.free_pages == c.pool.num_pages and (c.page_table.numpy() == -1).all()


def test_fused_projections_reseat_weights_and_fall_back():
    from torch import nn

    from compactattention_amd.prefill_sparse.llama.modeling_llama_common import FusedProjections

    torch.manual_seed(0)
    owner = nn.Module()
    owner.a = nn.Linear(16, 8, bias=False)
    owner.b = nn.Linear(16, 4, bias=False)
    ref_w = [owner.a.weight.detach().clone(), owner.b.weight.detach().clone()]
    fused = FusedProjections(owner, ("a", "b"))
    # the parameters are row blocks of one store, values and state_dict keys unchanged
    assert fused.intact()
    assert owner.a.weight.data_ptr() == fused.store.data_ptr()
    assert owner.b.weight.data_ptr() == fused.store.data_ptr() + 8 * 16 * 4
    assert torch.equal(owner.a.weight, ref_w[0]) and torch.equal(owner.b.weight, ref_w[1])
    assert sorted(owner.state_dict()) == ["a.weight", "b.weight"]
    x = torch.randn(3, 5, 16)
    ya, yb = fused(x)
    assert ya.shape == (3, 5, 8) and yb.shape == (3, 5, 4)
    assert torch.allclose(ya, x @ ref_w[0].T, atol=1e-5) and torch.allclose(yb, x @ ref_w[1].T, atol=1e-5)
    # in-place updates (init, load_state_dict) write through the views
    with torch.no_grad():
        owner.b.weight.mul_(2.0)
    assert torch.allclose(fused(x)[1], x @ (2 * ref_w[1]).T, atol=1e-5)
    # a replaced module is no longer backed by the store: the modules run one by one
    owner.b = nn.Linear(16, 4, bias=False)
    assert not fused.intact()
    assert torch.allclose(fused(x)[1], owner.b(x))
    fused.refuse()
    assert fused.intact() and torch.allclose(fused(x)[1], x @ owner.b.weight.T, atol=1e-5)
    # a dtype change (Module.to) also falls back
    owner.to(torch.float64)
    assert not fused.intact()
    assert fused(x.double())[0].dtype == torch.float64


def test_paged_cache_reset_keeps_owned_pages():
    from compactattention_amd.kv_cache import PagedKVCache

    c = PagedKVCache(2, 1, 128, "cpu")
    c.reserve(128)
    k = torch.zeros((2, 70, 1, 128), dtype=torch.bfloat16)
    c.append_tokens(k, k)
    owned = c.page_table.numpy().copy()
    c.reset(keep_pages=True)
    assert c.length == 0 and np.array_equal(c.page_table.numpy(), owned)
    c.append_tokens(k, k)
    c.fork(0, 1)  # request 1 now shares request 0's two pages
    c.reset(keep_pages=True)
    pt = c.page_table.numpy()
    assert (pt == -1).all() and c.pool.free_pages == c.pool.num_pages  # the shared pages went back


def test_seer_config_defaults_follow_the_reference():
    """The reference's compactattn Seer layer: threshold 5e-4, no schedule, keep_recent_blocks 2,
    gate Qavg_Kmaxminavg without force_double (configuration_llama_seerattn.py:191,198-200;
    modeling_llama_seerattn_chunked_dense.py:199-210); no sink or local blocks."""
    c = SeerAttnLlamaConfig()
    assert c.seerattn_compactattn_threshold == 5e-4 and c.seerattn_compactattn_threshold_schedule is None
    assert c.seerattn_compactattn_keep_recent_blocks == 2
    assert (c.compactattn_sink_blocks, c.compactattn_local_blocks) == (0, 0)
    assert (c.seerattn_gate_type, c.seerattn_gate_force_double) == ("Qavg_Kmaxminavg", False)


def test_threshold_schedule_normalize_and_resolve(tmp_path):
    import json

    from compactattention_amd.prefill_sparse.llama.modeling_llama_seerattn_chunked_dense import (
        normalize_compactattn_threshold_schedule as norm, resolve_compactattn_threshold as resolve)

    assert norm(None) is None and resolve(None, 10 ** 6, 0.25) == 0.25
    entries = [{"max_kv_len": 65536, "threshold": 1e-3}, {"max_kv_len": 8192, "threshold": 5e-3}]
    s = norm(entries)
    assert [e["max_kv_len"] for e in s["entries"]] == [8192, 65536]
    assert resolve(s, 8192, 0.0) == 5e-3            # inclusive upper bound
    assert resolve(s, 8193, 0.0) == 1e-3
    assert resolve(s, 10 ** 6, 0.0) == 1e-3         # past the last band: the last entry
    # dict form with a lower bound, tuple form, JSON file form
    s = norm({"entries": [{"max_kv_len": 10, "threshold": -1.0}], "threshold_lower_bound": 2e-4})
    assert resolve(s, 5, 0.0) == 2e-4
    assert norm(({"max_kv_len": 10, "threshold": -1.0},))["entries"][0]["threshold"] == 0.0  # default floor 0
    f = tmp_path / "sched.json"
    f.write_text(json.dumps({"entries": entries}))
    assert norm(str(f)) == norm(entries)
    for bad, err in (({"x": 1}, "must contain an 'entries'"), ([], "non-empty list"),
                     ([{"max_kv_len": 0, "threshold": 1}], "invalid max_kv_len"),
                     ([{"threshold": 1}], "must contain 'max_kv_len'")):
        with pytest.raises(ValueError, match=err):
            norm(bad)
    with pytest.raises(TypeError):
        norm(3.0)
    with pytest.raises(TypeError):
        norm([1.0])


def test_seer_layer_rule_maps_keep_recent_and_schedule(monkeypatch):
    """The layer's selection rule: the schedule's threshold for the chunk's kv length, the last
    keep_recent_blocks KV blocks as local blocks beyond the chunk, and the reference's debug
    overrides of both (attention_forward_chunked_dense.py:115-124,141-148)."""
    from compactattention_amd.prefill_sparse.llama.modeling_llama_seerattn_chunked_dense import \
        LlamaSeerAttentionChunkedDense

    sched = [{"max_kv_len": 1024, "threshold": 0.01}, {"max_kv_len": 4096, "threshold": 0.2}]
    attn = LlamaSeerAttentionChunkedDense(tiny(seerattn_compactattn_threshold_schedule=sched,
                                               seerattn_compactattn_keep_recent_blocks=6), 0)
    r = attn._selection_rule(4, 1024)
    assert (r.threshold, r.local_blocks, r.sink_blocks) == (0.01, 2, 0)
    r = attn._selection_rule(16, 2048)
    assert (r.threshold, r.local_blocks) == (0.2, 0)
    monkeypatch.setenv("SEERATTN_DEBUG_COMPACTATTN_THRESHOLD_OVERRIDE", "0.5")
    monkeypatch.setenv("SEERATTN_DEBUG_COMPACTATTN_KEEP_RECENT_OVERRIDE", "9")
    r = attn._selection_rule(4, 1024)
    assert (r.threshold, r.local_blocks) == (0.5, 5)
    b = LlamaSeerAttentionChunkedDense(tiny(compactattn_sink_blocks=1, compactattn_local_blocks=7), 0)
    monkeypatch.delenv("SEERATTN_DEBUG_COMPACTATTN_KEEP_RECENT_OVERRIDE")
    assert (b._selection_rule(4, 1024).sink_blocks, b._selection_rule(4, 1024).local_blocks) == (1, 7)
