"""GPU tests of the compactattn Llama models (chunked prefill through the HIP kernels).

- dense chunked prefill (every chunk over the whole past) matches an fp32 CPU forward of
  the same weights;
- a Seer threshold below every score keeps every block, so its logits equal the dense
  run's bit for bit (the tables are the identity);
- for one layer and chunk, the tables the model builds equal the CPU oracle's (bit-exact)
  for both selectors, recomputed from the layer's own Q/K, and the layer's attention output
  is within the north-star tolerance of the oracle over those tables.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from compactattention_amd.chunked_prefill import run_chunked_prefill_once, synthetic_prompt
from compactattention_amd.prefill_sparse.llama import (SeerAttnLlamaChunkedDenseForCausalLM, SeerAttnLlamaConfig,
                                                       SeerAttnLlamaFlashPrefillCompactAttnForCausalLM)
from compactattention_amd.prefill_sparse.llama.modeling_llama_common import apply_rotary_pos_emb, project_qkv
from compactattention_amd.synthetic import BASELINE_SEER

from .util import bits, f32, oracle_gate_summaries, ref_seer_tables

pytestmark = pytest.mark.gpu

T, CHUNK = 1280, 256


def tiny_config(**kw) -> SeerAttnLlamaConfig:
    base = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                num_key_value_heads=2, max_position_embeddings=2048, seerattn_compactattn_threshold=0.02,
                seerattn_flashprefill_alpha=0.3)
    base.update(kw)
    return SeerAttnLlamaConfig(**base)


def _model(cls, gpu, qk_scale: float = 1.0, gate_scale: float = 1.0, **kw):
    m = cls(tiny_config(**kw), device=gpu)
    m.init_weights(seed=11)
    # larger projections than N(0, 0.02) give the tiny model selective (non-flat) block scores
    with torch.no_grad():
        for layer in m.model.layers:
            layer.self_attn.q_proj.weight.mul_(qk_scale)
            layer.self_attn.k_proj.weight.mul_(qk_scale)
            if hasattr(layer.self_attn, "attn_gate"):
                for lin in (layer.self_attn.attn_gate.mask_linear_q, layer.self_attn.attn_gate.mask_linear_k):
                    if lin is not None:
                        lin.weight.mul_(gate_scale)
    return m


def _reference_logits(model, input_ids: torch.Tensor) -> torch.Tensor:
    """fp32 CPU forward over the whole prompt with causal softmax attention."""
    c = model.config
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    ids = input_ids.cpu()
    h = sd["model.embed_tokens.weight"][ids]
    L = ids.shape[1]
    cos = model.model.rotary_emb.cos[:L].cpu()
    sin = model.model.rotary_emb.sin[:L].cpu()

    def rms(x, w):
        return w * F.rms_norm(x, (x.shape[-1],), eps=c.rms_norm_eps)

    for i in range(c.num_hidden_layers):
        p = f"model.layers.{i}."
        x = rms(h, sd[p + "input_layernorm.weight"])
        q = (x @ sd[p + "self_attn.q_proj.weight"].T).view(1, L, c.num_attention_heads, 128)
        k = (x @ sd[p + "self_attn.k_proj.weight"].T).view(1, L, c.num_key_value_heads, 128)
        v = (x @ sd[p + "self_attn.v_proj.weight"].T).view(1, L, c.num_key_value_heads, 128)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        g = c.num_key_value_groups
        kq = k.repeat_interleave(g, dim=2)
        vq = v.repeat_interleave(g, dim=2)
        s = torch.einsum("bqhd,bkhd->bhqk", q, kq) / math.sqrt(128)
        s = s.masked_fill(torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf"))
        o = torch.einsum("bhqk,bkhd->bqhd", torch.softmax(s, -1), vq).reshape(1, L, -1)
        h = h + o @ sd[p + "self_attn.o_proj.weight"].T
        x = rms(h, sd[p + "post_attention_layernorm.weight"])
        mlp = F.silu(x @ sd[p + "mlp.gate_proj.weight"].T) * (x @ sd[p + "mlp.up_proj.weight"].T)
        h = h + mlp @ sd[p + "mlp.down_proj.weight"].T
    h = rms(h, sd["model.norm.weight"])
    return h[:, -1:] @ sd["lm_head.weight"].T


def test_dense_prefill_matches_fp32_reference(gpu):
    print("case: model dense vs fp32", flush=True)
    m = _model(SeerAttnLlamaChunkedDenseForCausalLM, gpu, seerattn_chunked_prefill_force_dense=True)
    ids = synthetic_prompt(1, T, m.config.vocab_size, 1234, gpu)
    logits, _ = run_chunked_prefill_once(m, ids, CHUNK)
    ref = _reference_logits(m, ids)
    got = logits.float().cpu()
    cos = F.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
    assert cos > 0.999, cos
    assert (got - ref).abs().max().item() <= 0.05 * ref.abs().max().item()


def test_seer_keep_all_equals_dense(gpu):
    print("case: model keep-all vs dense", flush=True)
    ids = synthetic_prompt(1, T, 512, 99, gpu)
    dense = _model(SeerAttnLlamaChunkedDenseForCausalLM, gpu, seerattn_chunked_prefill_force_dense=True)
    keep_all = _model(SeerAttnLlamaChunkedDenseForCausalLM, gpu, seerattn_compactattn_threshold=-1.0)
    a, _ = run_chunked_prefill_once(dense, ids, CHUNK)
    b, _ = run_chunked_prefill_once(keep_all, ids, CHUNK)
    assert torch.equal(a, b)


@pytest.mark.parametrize("cls", [SeerAttnLlamaChunkedDenseForCausalLM, SeerAttnLlamaFlashPrefillCompactAttnForCausalLM])
def test_decode_steps_match_fp32_reference(gpu, cls):
    """Dense chunked prefill, then decode steps of 1, 5 and 1 tokens from an unaligned cache
    length: each step's last logits match the fp32 CPU forward over the whole sequence."""
    print(f"case: model decode {cls.__name__}", flush=True)
    m = _model(cls, gpu, seerattn_chunked_prefill_force_dense=True)
    ids = synthetic_prompt(1, T + 7, m.config.vocab_size, 4321, gpu)
    cache = m.new_cache(1, T + 64)
    for s0 in range(0, T, CHUNK):
        m(ids[:, s0:s0 + CHUNK], cache)
    pos = T
    for n in (1, 5, 1):
        logits = m(ids[:, pos:pos + n], cache)
        pos += n
        assert cache.get_seq_length() == pos
        ref = _reference_logits(m, ids[:, :pos])
        got = logits.float().cpu()
        cos = F.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
        assert cos > 0.999, (n, cos)
        assert (got - ref).abs().max().item() <= 0.05 * ref.abs().max().item()
    with pytest.raises(ValueError, match="at most 64"):  # after decode steps every call is a decode step
        m(ids[:, :128], cache)


@pytest.mark.parametrize("cls", [SeerAttnLlamaChunkedDenseForCausalLM, SeerAttnLlamaFlashPrefillCompactAttnForCausalLM])
def test_paged_cache_growth_matches_reserved_cache(gpu, cls):
    """A selecting prefill into a cache reserved for 128 tokens (the page pool, the page tables
    and the summaries grow during the run, pages land wherever the allocator puts them) gives
    the same logits bit for bit as one into a cache reserved for the whole prompt, and the
    page tables are not the identity."""
    print(f"case: model cache growth {cls.__name__}", flush=True)
    m = _model(cls, gpu, qk_scale=8.0, gate_scale=20.0, seerattn_compactattn_threshold=0.1)
    ids = synthetic_prompt(1, T, m.config.vocab_size, 5150, gpu)
    big = m.new_cache(1, T)
    small = m.new_cache(1, 128)
    pool0 = small.layer(0).pool.num_pages
    a, _ = run_chunked_prefill_once(m, ids, CHUNK, big)
    b, _ = run_chunked_prefill_once(m, ids, CHUNK, small)
    assert torch.equal(a, b)
    lay = small.layer(1)
    assert lay.pool.num_pages > pool0 and lay.cap >= T // 64
    pt = lay.page_table[:, :T // 64].cpu()
    ident = torch.arange(T // 64, dtype=torch.int32)[None, :] + (T // 64) * torch.arange(pt.shape[0])[:, None]
    assert (pt >= 0).all() and not torch.equal(pt, ident.to(torch.int32))
    assert torch.equal(lay.k_hf(), big.layer(1).k_hf())


@pytest.mark.parametrize("cls", [SeerAttnLlamaChunkedDenseForCausalLM, SeerAttnLlamaFlashPrefillCompactAttnForCausalLM])
def test_unaligned_prompt_matches_fp32_reference(gpu, cls):
    """A prompt of 64*n + 37 tokens: the last chunk's aligned part takes the chunk path and its
    37-token tail one dense decode step; the last logits match the fp32 CPU forward, a decode
    step continues from the unaligned length, and a keep-all Seer selection equals the dense
    run bit for bit."""
    print(f"case: model unaligned prompt {cls.__name__}", flush=True)
    n = T + 37
    m = _model(cls, gpu, seerattn_chunked_prefill_force_dense=True)
    ids = synthetic_prompt(1, n + 1, m.config.vocab_size, 2024, gpu)
    cache = m.new_cache(1, n + 64)
    logits, _ = run_chunked_prefill_once(m, ids[:, :n], CHUNK, cache)
    assert cache.get_seq_length() == n
    for upto, got in ((n, logits), (n + 1, m(ids[:, n:n + 1], cache))):
        ref = _reference_logits(m, ids[:, :upto])
        got = got.float().cpu()
        cos = F.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
        assert cos > 0.999, (upto, cos)
        assert (got - ref).abs().max().item() <= 0.05 * ref.abs().max().item()
    if cls is SeerAttnLlamaChunkedDenseForCausalLM:
        keep_all = _model(cls, gpu, seerattn_compactattn_threshold=-1.0)
        b, _ = run_chunked_prefill_once(keep_all, ids[:, :n], CHUNK)
        assert torch.equal(logits, b)


@pytest.mark.parametrize("variant", ["seer_compactattn", "flashprefill_compactattn"])
def test_hf_replacement_matches_stock_model(gpu, variant):
    """A stock transformers Llama with its attention replaced (dense chunks, then decode steps)
    matches the same stock model run in fp32 on the CPU with its own attention."""
    import copy

    transformers = pytest.importorskip("transformers")
    from compactattention_amd.load_attention_replacement import (load_llama_attention_replacement_model,
                                                                 new_compactattn_cache)

    print(f"case: hf replacement {variant}", flush=True)
    cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                                   max_position_embeddings=2048)
    torch.manual_seed(11)
    stock = transformers.LlamaForCausalLM(cfg).eval()
    ref_model = copy.deepcopy(stock).float()
    model = load_llama_attention_replacement_model(base_model=stock.to(gpu), variant=variant)
    model.compactattn_config.seerattn_chunked_prefill_force_dense = True
    ids = synthetic_prompt(1, T + 6, cfg.vocab_size, 77, gpu)
    cache = new_compactattn_cache(model, 1, T + 64)

    def check(logits, upto):
        with torch.no_grad():
            ref = ref_model(input_ids=ids[:, :upto].cpu()).logits[:, -1:].float()
        got = logits.float().cpu()
        cos = F.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
        assert cos > 0.999, (upto, cos)
        assert (got - ref).abs().max().item() <= 0.05 * ref.abs().max().item()

    logits, _ = run_chunked_prefill_once(model, ids[:, :T], CHUNK, cache)
    check(logits, T)
    pos = T
    for n in (1, 5):
        with torch.no_grad():
            logits = model(input_ids=ids[:, pos:pos + n], past_key_values=cache, use_cache=True,
                           logits_to_keep=1).logits
        pos += n
        check(logits, pos)
    # the selecting path runs through the same adapter: later chunks select blocks
    model.compactattn_config.seerattn_chunked_prefill_force_dense = False
    for layer in model.model.layers:
        layer.self_attn.compactattn_debug = True
    logits, _ = run_chunked_prefill_once(model, ids[:, :T], CHUNK, cache)
    assert torch.isfinite(logits.float()).all()
    stats = model.model.layers[1].self_attn._compactattn_last_stats
    assert stats["path"] in ("chunked_selected", "flashprefill_chunked_selected")


def _capture_layer_inputs(model, layer_idx):
    captured = []
    attn = model.model.layers[layer_idx].self_attn
    handle = attn.register_forward_pre_hook(lambda mod, args: captured.append(args[0].detach().clone()))
    attn.compactattn_debug = True
    return captured, handle, attn


def _layer_qkv(attn, hidden, start, model):
    B, L, _ = hidden.shape
    q, k, v = project_qkv(attn, hidden)  # the layer's own (fused) projection GEMM
    cos, sin = model.model.rotary_emb.tokens(start, L)
    qr, kr = apply_rotary_pos_emb(q, k, cos, sin)
    return q, k, v, qr, kr


SEER_GATES = {
    # the reference's default gate (no query projection, W_k [Hq, 384, 128] on max/min/avg K) and
    # the reference's rule: threshold + the last keep_recent_blocks KV blocks
    "seer": {},
    # keep_recent_blocks beyond the chunk's 4 blocks: the 3 past blocks before it are forced
    "seer_keep_recent_7": dict(seerattn_compactattn_keep_recent_blocks=7),
    "seer_kv_aware_gate": dict(seerattn_compactattn_kv_group_aware_gate=True),
    # BASELINE configs 1 and 3: Qavg_Kavg with force_double, threshold + sink + 2 local blocks
    "seer_baseline": dict(BASELINE_SEER, seerattn_compactattn_threshold=0.1),
}


@pytest.mark.parametrize("selector", ["seer", "seer_keep_recent_7", "seer_kv_aware_gate", "seer_baseline",
                                      "flashprefill", "flashprefill_128", "seer_tail37", "flashprefill_tail37"])
def test_layer_tables_bit_exact(gpu, selector):
    """Per layer, the tables the model builds for its last chunk equal the reference's
    selection recomputed from the layer's own inputs: for the Seer layer the restatement of the
    reference's rule (tests/util.ref_seer_tables) on the oracle's gate scores; for BASELINE's
    sink + local variant and FlashPrefill the oracle's rule.  The _tail37 cases end the prompt
    with a 37-token chunk, which selects with one partial query and key block."""
    print(f"case: model layer tables {selector}", flush=True)
    seer = selector.startswith("seer")
    tlen = T + (37 if selector.endswith("_tail37") else 0)
    cls = SeerAttnLlamaChunkedDenseForCausalLM if seer else SeerAttnLlamaFlashPrefillCompactAttnForCausalLM
    kw = dict(seerattn_compactattn_threshold=0.1,
              seerattn_flashprefill_block_size=128 if selector == "flashprefill_128" else 64)
    kw.update(SEER_GATES.get(selector, {}))
    m = _model(cls, gpu, qk_scale=8.0 if seer else 40.0, gate_scale=20.0, **kw)
    layer_idx = 1
    captured, handle, attn = _capture_layer_inputs(m, layer_idx)
    ids = synthetic_prompt(1, tlen, m.config.vocab_size, 7, gpu)
    with torch.no_grad():
        run_chunked_prefill_once(m, ids, CHUNK)
    handle.remove()
    stats = attn._compactattn_last_stats
    last_len = tlen - CHUNK * ((tlen - 1) // CHUNK)
    assert stats["past_blocks"] == (tlen - last_len) // 64
    with torch.no_grad():
        parts = [_layer_qkv(attn, h, i * CHUNK, m) for i, h in enumerate(captured)]
    q_nope, k_nope, _, q_rope, _ = parts[-1]
    k_nope_all = torch.cat([p[1] for p in parts], dim=1)
    k_rope_all = torch.cat([p[4] for p in parts], dim=1)
    v_all = torch.cat([p[2] for p in parts], dim=1)
    P = [stats["past_blocks"]]
    Hkv = m.config.num_key_value_heads
    c = m.config
    table = counts = None
    if seer:
        bcos, bsin = (f32(t) for t in m.model.rotary_emb.blocks())
        qhat, khat = oracle_gate_summaries(attn.attn_gate, bits(q_nope), bits(k_nope_all), bcos, bsin, P[0])
        scores = oracle.block_scores(qhat, khat, P, 128 ** -0.5)
        if selector == "seer_baseline":
            rule = oracle.Rule(threshold=0.1, sink_blocks=1, local_blocks=2)
            last_n = 0
        else:
            table, counts = ref_seer_tables(scores, P, Hkv, 0.1, c.seerattn_compactattn_keep_recent_blocks,
                                            kv_group_aware=c.seerattn_compactattn_kv_group_aware_gate)
    else:
        qhat = oracle.block_mean(bits(q_rope))
        khat = oracle.block_mean(bits(k_rope_all))
        rule = oracle.Rule(topk=c.seerattn_flashprefill_min_budget, alpha=c.seerattn_flashprefill_alpha,
                           sink_blocks=c.seerattn_flashprefill_attention_sink,
                           window_blocks=c.seerattn_flashprefill_window_size,
                           last_n_block=c.seerattn_flashprefill_last_n_block, topk_all_columns=True)
        last_n = c.seerattn_flashprefill_last_n_block
        if selector == "flashprefill_128":  # 128-token score blocks, then both 64-token pages of each
            P128 = [P[0] // 2]
            scores = oracle.block_scores(oracle.pair_block_means(qhat, 64), oracle.pair_block_means(khat, 64), P128,
                                         1.0 / math.sqrt(128))
            _, _, t128, c128 = oracle.union_compact(oracle.select_rows(scores, P128, rule), Hkv, P128, last_n)
            cap64 = P[0] + CHUNK // 64
            table = np.full((Hkv, cap64), -1, np.int32)
            counts = np.zeros((Hkv,), np.int32)
            for r in range(Hkv):
                pages = [2 * kb + i for kb in t128[r, :c128[r]] for i in (0, 1)]
                table[r, :len(pages)] = pages
                counts[r] = len(pages)
        else:
            scores = oracle.block_scores(qhat, khat, P, 1.0 / math.sqrt(128))
    if table is None:
        keep = oracle.select_rows(scores, P, rule)
        _, _, table, counts = oracle.union_compact(keep, Hkv, P, last_n)
    got_counts = stats["counts"].cpu().numpy()
    got_table = stats["table"].cpu().numpy()
    assert np.array_equal(got_counts, counts)
    assert np.array_equal(got_table[:, :table.shape[1]], table)
    nkb = P[0] + -(-last_len // 64)
    assert counts.min() < nkb, "the test wants a selective layer (some blocks dropped)"
    if selector == "seer_keep_recent_7":
        for r in range(Hkv):
            assert {P[0] - 3, P[0] - 2, P[0] - 1} <= set(table[r, :counts[r]].tolist())
    # attention over the selected pages, recomputed from the layer's own inputs (the oracle's key
    # arrays padded to whole blocks; a query never sees the padding)
    kc = k_rope_all.transpose(1, 2).contiguous()
    vc = v_all.transpose(1, 2).contiguous()
    pad = (0, 0, 0, 64 * nkb - kc.shape[2])
    ref = oracle.attention(bits(q_rope), bits(F.pad(kc, pad)), bits(F.pad(vc, pad)), P, table[:, :nkb], counts,
                           128 ** -0.5)
    out = torch.empty_like(q_rope)
    from compactattention_amd import ops
    ops.attn_fwd(q_rope, ops.KV.heads_first(kc), ops.KV.heads_first(vc), stats["table"], stats["counts"], P,
                 128 ** -0.5, nkb, Hkv, out=out)
    err = np.abs(f32(out) - ref)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())


def _seer_last_chunk_scores(attn, captured, block_rope, project):
    """The oracle's gate scores of a Seer layer's last chunk, recomputed from the hidden states
    the layer received (``captured``, one per chunk) through its own q/k projections."""
    parts = [project(attn, h) for h in captured]
    q_nope = parts[-1][0]
    k_nope_all = torch.cat([p[1] for p in parts], dim=1)
    P = [(k_nope_all.shape[1] - q_nope.shape[1]) // 64]
    bcos, bsin = (f32(t) for t in block_rope)
    qhat, khat = oracle_gate_summaries(attn.attn_gate, bits(q_nope), bits(k_nope_all), bcos, bsin, P[0])
    return oracle.block_scores(qhat, khat, P, 128 ** -0.5), P


def test_threshold_schedule_bands(gpu):
    """seerattn_compactattn_threshold_schedule: the layer looks its threshold up by the chunk's
    kv length (modeling_llama_seerattn_chunked_dense.py:36-98,225-227,871): a chunk ending at
    1024 tokens takes the <= 1024 band's threshold, one ending at 1280 the <= 4096 band's; the
    tables equal the reference's rule at that threshold and differ between the bands."""
    print("case: model threshold schedule", flush=True)
    sched = {"entries": [{"max_kv_len": 4096, "threshold": 0.3}, {"max_kv_len": 1024, "threshold": 0.02}]}
    m = _model(SeerAttnLlamaChunkedDenseForCausalLM, gpu, qk_scale=8.0, gate_scale=20.0,
               seerattn_compactattn_threshold=0.9, seerattn_compactattn_threshold_schedule=sched)
    ids = synthetic_prompt(1, T, m.config.vocab_size, 7, gpu)
    Hkv = m.config.num_key_value_heads
    results = []
    for upto, thr in ((1024, 0.02), (1280, 0.3)):
        captured, handle, attn = _capture_layer_inputs(m, 1)
        with torch.no_grad():
            run_chunked_prefill_once(m, ids[:, :upto], CHUNK)
        handle.remove()
        with torch.no_grad():
            scores, P = _seer_last_chunk_scores(attn, captured, m.model.rotary_emb.blocks(),
                                                lambda a, h: project_qkv(a, h)[:2])
        table, counts = ref_seer_tables(scores, P, Hkv, thr, 2)
        stats = attn._compactattn_last_stats
        assert np.array_equal(stats["counts"].cpu().numpy(), counts), upto
        assert np.array_equal(stats["table"].cpu().numpy()[:, :table.shape[1]], table), upto
        other, _ = ref_seer_tables(scores, P, Hkv, 0.3 if thr == 0.02 else 0.02, 2)
        assert not np.array_equal(other, table), "the two bands should select differently"
        results.append(counts)


def test_hf_replacement_layer_tables_reference_rule(gpu):
    """The stock-transformers replacement (seer_compactattn, the reference's default gate, no
    sink or local blocks, keep_recent_blocks 2 and 6): the tables of a layer's last chunk equal
    the reference's rule recomputed from the layer's inputs."""
    transformers = pytest.importorskip("transformers")
    from compactattention_amd.load_attention_replacement import (load_llama_attention_replacement_model,
                                                                 new_compactattn_cache)

    cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                                   max_position_embeddings=2048)
    for keep_recent in (2, 6):
        print(f"case: hf replacement tables keep_recent={keep_recent}", flush=True)
        torch.manual_seed(12)
        stock = transformers.LlamaForCausalLM(cfg).eval()
        with torch.no_grad():
            for layer in stock.model.layers:
                layer.self_attn.q_proj.weight.mul_(40.0)
                layer.self_attn.k_proj.weight.mul_(40.0)
        model = load_llama_attention_replacement_model(base_model=stock.to(gpu), variant="seer_compactattn",
                                                       threshold=0.05, compactattn_keep_recent_blocks=keep_recent)
        attn = model.model.layers[1].self_attn
        c = model.compactattn_config
        assert (c.compactattn_sink_blocks, c.compactattn_local_blocks) == (0, 0)
        assert c.seerattn_gate_type == "Qavg_Kmaxminavg" and not c.seerattn_gate_force_double
        with torch.no_grad():
            attn.attn_gate.mask_linear_k.weight.mul_(20.0)
        captured = []
        handle = attn.register_forward_pre_hook(
            lambda mod, args, kwargs: captured.append(kwargs["hidden_states"].detach().clone()), with_kwargs=True)
        attn.compactattn_debug = True
        ids = synthetic_prompt(1, T, cfg.vocab_size, 8, gpu)
        cache = new_compactattn_cache(model, 1, T)
        with torch.no_grad():
            run_chunked_prefill_once(model, ids, CHUNK, cache)
            handle.remove()
            scores, P = _seer_last_chunk_scores(attn, captured, model.compactattn_block_rope.get(gpu),
                                                lambda a, h: project_qkv(a, h)[:2])
        table, counts = ref_seer_tables(scores, P, c.num_key_value_heads, 0.05, keep_recent)
        stats = attn._compactattn_last_stats
        assert stats["path"] == "chunked_selected"
        assert np.array_equal(stats["counts"].cpu().numpy(), counts)
        assert np.array_equal(stats["table"].cpu().numpy()[:, :table.shape[1]], table)
        assert counts.min() < P[0] + CHUNK // 64, "the test wants a selective layer"
