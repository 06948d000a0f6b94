"""BASELINE configs at their full sizes (and config 3's attention shape) on the GPU.

Config 2: a 131072-token paged heads-first cache, a 1024-token chunk, 32 Q / 8 KV heads,
FlashPrefill pooled top-k (k = 10, about a quarter of the past after the union) + sink block 0
+ 2 local blocks, and the 10 % and 50 % points of the keep sweep.  Config 0: 256 queries over
8192 keys.  Config 1: AttnGate at 32768 tokens.  Config 3's layer shape: a 2048-token chunk
at the end of a 131072-token prompt.  Config 4: the ragged four-request batch at G = 7.

The selection path is integer/fp32 work with a fixed evaluation order, so at these sizes it
is still checked bit for bit against the CPU oracle (which runs it in well under a second):
block means, pooled queries, per-row masks, the GQA union, tables and counts.  The attention
output is checked on every query row of every head against an fp32 torch attention on the
GPU over the same selected blocks (tests/util.torch_reference_check: gathered K/V, causal
mask, softmax, PV -- no code shared with the kernel or the oracle), at the north-star
tolerance (max-abs 2e-2, mean-abs 2e-3), and so is the log-sum-exp; a few rows are also
checked against the fp64 C oracle, which ties the two references together.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from compactattention_amd import ops
from compactattention_amd.synthetic import make_chunk, make_chunk_device

from .util import bits, f32, float_bits_equal, torch_reference_check, unpack_rowmask

pytestmark = pytest.mark.gpu

PAST, LQ, HQ, HKV = 131072, 1024, 32, 8
TOPK = 10
ATOL_MAX = 2e-2
ATOL_MEAN = 2e-3
SCALE = 1.0 / math.sqrt(128)


def _fill(ch, K, V, kmean, past: int, lq: int, step: int = 16384, **gate):
    """The cache-fill kernel appends the past in pieces, then the chunk (the path's append)."""
    for t0 in range(0, past, step):
        t1 = min(past, t0 + step)
        ops.cache_fill(ch.k[:, :, t0:t1].transpose(1, 2).contiguous(), ch.v[:, :, t0:t1].transpose(1, 2).contiguous(),
                       K, V, [t0 // 64], ch.kv_cap, kmean, **gate)
    ops.cache_fill(ch.k[:, :, past:past + lq].transpose(1, 2).contiguous(),
                   ch.v[:, :, past:past + lq].transpose(1, 2).contiguous(), K, V, [past // 64], ch.kv_cap, kmean,
                   **gate)


def _oracle_scores(ch):
    """Oracle pooled scores of a single-request chunk from the oracle's own block means."""
    P = ch.past_blocks
    nkb = P[0] + ch.q.shape[1] // 64
    hkv = ch.k.shape[1]
    khat_ref = oracle.block_mean(np.ascontiguousarray(bits(ch.k)[:, :, :nkb * 64].transpose(0, 2, 1, 3)))
    khat = np.zeros((1, hkv, ch.kv_cap, 128), dtype=np.float32)
    khat[:, :, :nkb] = khat_ref
    qhat_ref = oracle.block_mean(bits(ch.q))
    return khat_ref, qhat_ref, oracle.block_scores(qhat_ref, khat, P, SCALE)


def _select(qhat, kmean, P, hkv, cap, topk):
    rule = ops.Rule(topk=topk, sink_blocks=1, local_blocks=2)
    rowmask, _ = ops.score_select(qhat, kmean, SCALE, rule, P, hkv, cap)
    table, counts, _, _ = ops.union_compact(rowmask, P, hkv, cap)
    return rowmask, table, counts


def _keep_ratio(counts, P, qb):
    return float((counts.float() - qb).mean().item()) / P


def _calibrate(qhat, kmean, P, hkv, cap, qb, target):
    """The top-k whose post-union past keep ratio is closest to target (as the bench does)."""
    best = None
    for k in (1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 20, 24, 28, 32, 40, 48, 56, 64):
        _, _, counts = _select(qhat, kmean, P, hkv, cap, k)
        r = _keep_ratio(counts, P[0], qb)
        if best is None or abs(r - target) < abs(best[1] - target):
            best = (k, r)
    return best


def _check_tables(rowmask, table, counts, sc, P, hkv, cap, topk):
    keep = oracle.select_rows(sc, P, oracle.Rule(topk=topk, sink_blocks=1, local_blocks=2))
    assert np.array_equal(unpack_rowmask(rowmask, cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, hkv, P)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)


def _check_attention(q, kc, vc, P, table, counts, cap, hkv, oracle_rows=((0, 4),), **kw):
    """All rows against the fp32 torch reference; a few rows against the fp64 C oracle."""
    out, lse = ops.attn_fwd(q, ops.KV.heads_first(kc), ops.KV.heads_first(vc), table, counts, P, SCALE, cap, hkv,
                            with_lse=True, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    torch_reference_check(out, q, kc, vc, P, table, counts, SCALE, lse=lse)
    got = f32(out)
    tab, cnt = table.cpu().numpy(), counts.cpu().numpy()
    for q0, q1 in oracle_rows:
        ref = oracle.attention(bits(q), bits(kc), bits(vc), P, tab, cnt, SCALE, q_range=(q0, q1))
        err = np.abs(got[:, q0:q1] - ref[:, q0:q1])
        assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (q0, err.max(), err.mean())
    return out


# ----------------------------------------------------------------------------- config 2
@pytest.fixture(scope="module")
def full(gpu):
    print("case: full-size config 2 (131072 past tokens, chunk 1024, 32/8 heads)", flush=True)
    ch = make_chunk_device(PAST, LQ, HQ, HKV, gpu)
    cap, P = ch.kv_cap, ch.past_blocks
    kc, vc = torch.zeros_like(ch.k), torch.zeros_like(ch.v)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((HKV, cap, 128), dtype=torch.float32, device=gpu)
    _fill(ch, K, V, kmean, PAST, LQ)
    qhat = ops.pool_query(ch.q, P, cap)
    rowmask, table, counts = _select(qhat, kmean, P, HKV, cap, TOPK)
    torch.cuda.synchronize()
    khat_ref, qhat_ref, sc = _oracle_scores(ch)
    return dict(ch=ch, cap=cap, P=P, K=K, V=V, kc=kc, vc=vc, kmean=kmean, qhat=qhat, rowmask=rowmask,
                table=table, counts=counts, khat_ref=khat_ref, qhat_ref=qhat_ref, sc=sc)


def test_fullsize_cache_and_selection_bit_exact(full):
    ch, cap, P = full["ch"], full["cap"], full["P"]
    nkb = P[0] + LQ // 64
    # the cache holds the appended tokens unchanged
    assert torch.equal(full["kc"][:, :, :nkb * 64].view(torch.int16), ch.k[:, :, :nkb * 64].view(torch.int16))
    assert torch.equal(full["vc"][:, :, :nkb * 64].view(torch.int16), ch.v[:, :, :nkb * 64].view(torch.int16))
    # block means of every cached block, pooled queries, per-row masks, union and tables
    assert float_bits_equal(f32(full["kmean"][:, :nkb]).reshape(1, HKV, nkb, 128), full["khat_ref"])
    assert float_bits_equal(f32(full["qhat"]), full["qhat_ref"])
    _check_tables(full["rowmask"], full["table"], full["counts"], full["sc"], P, HKV, cap, TOPK)


def test_fullsize_table_structure(full):
    P, cap = full["P"][0], full["cap"]
    qb = LQ // 64
    table = full["table"].cpu().numpy()
    counts = full["counts"].cpu().numpy()
    for r in range(HKV):
        n = int(counts[r])
        row = table[r, :n]
        assert qb < n <= P + qb
        assert (np.diff(row) > 0).all()  # strictly ascending, unique
        assert np.array_equal(row[-qb:], np.arange(P, P + qb))  # the chunk's blocks close the row
        assert row[0] == 0  # sink block
        assert {P - 2, P - 1} <= set(row.tolist())  # the 2 local blocks
        # every query row keeps at least top-k past blocks, so the union keeps at least k
        assert n - qb >= TOPK
    keep = (counts - qb).sum() / (HKV * P)
    assert 0.15 < keep < 0.40, keep  # the planted inputs give about a quarter at k = 10


def test_fullsize_attention_all_rows(full):
    """Every query row of every head at 128K cached tokens (the automatic plan)."""
    ch, P, cap = full["ch"], full["P"], full["cap"]
    _check_attention(ch.q, full["kc"], full["vc"], P, full["table"], full["counts"], cap, HKV,
                     oracle_rows=((0, 4), (LQ - 4, LQ)))


@pytest.mark.parametrize("forced", [1, 3])
def test_fullsize_split_plan_matches_unsplit(full, forced):
    """The automatic split plan against forced split counts (1: no partials; 3: three
    partials per row merged by LSE)."""
    ch, P, cap = full["ch"], full["P"], full["cap"]
    args = (ch.q, full["K"], full["V"], full["table"], full["counts"], P, SCALE, cap, HKV)
    auto = ops.attn_fwd(*args, num_splits=0)
    other = ops.attn_fwd(*args, num_splits=forced)
    torch.cuda.synchronize()
    # the split plan changes only where the online softmax rescales and the merge's rounding:
    # a few bf16 ulps at most, on a small share of the outputs
    d = (other.float() - auto.float()).abs()
    assert d.max().item() <= ATOL_MAX and d.mean().item() <= 2e-4, (d.max().item(), d.mean().item())


@pytest.mark.parametrize("target", [0.10, 0.50])
def test_fullsize_keep_sweep_points(full, target):
    """The bench's 10 % and 50 % keep points: top-k calibrated like the bench, tables bit-exact
    against the oracle, every attention row against the fp32 torch reference."""
    print(f"case: full-size config 2 sweep point {target}", flush=True)
    ch, P, cap = full["ch"], full["P"], full["cap"]
    qb = LQ // 64
    topk, ratio = _calibrate(full["qhat"], full["kmean"], P, HKV, cap, qb, target)
    assert abs(ratio - target) < 0.06, (topk, ratio)
    rowmask, table, counts = _select(full["qhat"], full["kmean"], P, HKV, cap, topk)
    _check_tables(rowmask, table, counts, full["sc"], P, HKV, cap, topk)
    _check_attention(ch.q, full["kc"], full["vc"], P, table, counts, cap, HKV)


# ----------------------------------------------------------------------------- config 0
def test_config0_shape(gpu):
    """Config 0 (BASELINE's CPU-runnable case) on the HIP path: 256 queries over 8192 keys
    (P = 124, C = 4), 32 / 8 heads, planted inputs (seed 1234, 8 blocks per KV head get +2.0
    along a shared direction), FlashPrefill pooled top-k + sink block 0 + 2 local blocks at
    about 25 % post-union keep.  Tables bit-exact against the oracle, attention on every row,
    and the planted blocks recalled by the HIP tables far above the keep ratio."""
    print("case: config 0 (256 queries over 8192 keys, 32/8 heads)", flush=True)
    lq, hq, hkv = 256, 32, 8
    ch = make_chunk([8192 - lq], lq, hq, hkv, seed=1234)
    P, cap = ch.past_blocks, ch.kv_cap
    kc, vc = torch.zeros_like(ch.k, device=gpu), torch.zeros_like(ch.v, device=gpu)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((hkv, cap, 128), dtype=torch.float32, device=gpu)
    dev = type(ch)(ch.q.to(gpu), ch.k.to(gpu), ch.v.to(gpu), ch.past_blocks, ch.kv_cap, ch.planted)
    _fill(dev, K, V, kmean, P[0] * 64, lq)
    qhat = ops.pool_query(dev.q, P, cap)
    topk, ratio = _calibrate(qhat, kmean, P, hkv, cap, lq // 64, 0.25)
    assert 0.2 <= ratio <= 0.3, (topk, ratio)
    rowmask, table, counts = _select(qhat, kmean, P, hkv, cap, topk)
    _, _, sc = _oracle_scores(ch)
    _check_tables(rowmask, table, counts, sc, P, hkv, cap, topk)
    _check_attention(dev.q, kc, vc, P, table, counts, cap, hkv, oracle_rows=((0, lq),))
    tab, cnt = table.cpu().numpy(), counts.cpu().numpy()
    hits = sum(int(blk in set(tab[h, :cnt[h]].tolist())) for h in range(hkv) for blk in ch.planted[0][h])
    recall = hits / sum(len(p) for p in ch.planted[0])
    assert recall >= 0.5, (recall, ratio)


# ----------------------------------------------------------------------------- config 1
def test_fullsize_config1_attngate(gpu):
    """Config 1: 32768 cached tokens of which the last 1024 are the chunk (P = 496), 32 / 8
    heads, AttnGate (mean-pooled Q and K, per-head 128x128 projections ~ N(0, 0.02), block
    RoPE), softmax threshold 5e-3 + sink block + 2 local blocks."""
    from compactattention_amd.synthetic import rope_tables

    print("case: full-size config 1 (AttnGate, 32768 tokens, chunk 1024)", flush=True)
    past, lq, hq, hkv = 31744, 1024, 32, 8
    ch = make_chunk_device(past, lq, hq, hkv, gpu)
    cap, P = ch.kv_cap, ch.past_blocks
    g = torch.Generator().manual_seed(1234)
    wq = (torch.randn((hq, 128, 128), generator=g) * 0.02).float()
    wk = (torch.randn((hkv, 128, 128), generator=g) * 0.02).float()
    cos, sin = rope_tables(cap)
    kc, vc = torch.zeros_like(ch.k), torch.zeros_like(ch.v)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((hkv, cap, 128), dtype=torch.float32, device=gpu)
    kgate = torch.zeros_like(kmean)
    _fill(ch, K, V, kmean, past, lq, gate_wk=wk.to(gpu), rope_cos=cos.to(gpu), rope_sin=sin.to(gpu), kgate=kgate)
    rule = ops.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2)
    qhat = ops.pool_query(ch.q, P, cap, gate_wq=wq.to(gpu), rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
    rowmask, _ = ops.score_select(qhat, kgate, SCALE, rule, P, hkv, cap)
    table, counts, _, _ = ops.union_compact(rowmask, P, hkv, cap)
    torch.cuda.synchronize()
    nkb = P[0] + lq // 64
    means = oracle.block_mean(np.ascontiguousarray(bits(ch.k)[:, :, :nkb * 64].transpose(0, 2, 1, 3)))
    khat = np.zeros((1, hkv, cap, 128), dtype=np.float32)
    khat[:, :, :nkb] = oracle.gate_project(means, f32(wk), f32(cos), f32(sin), [0])
    assert float_bits_equal(f32(kgate[:, :nkb]).reshape(1, hkv, nkb, 128), khat[:, :, :nkb])
    qref = oracle.gate_project(oracle.block_mean(bits(ch.q)), f32(wq), f32(cos), f32(sin), P)
    assert float_bits_equal(f32(qhat), qref)
    keep = oracle.select_rows(oracle.block_scores(qref, khat, P, SCALE), P,
                              oracle.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2))
    assert np.array_equal(unpack_rowmask(rowmask, cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, hkv, P)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)
    _check_attention(ch.q, kc, vc, P, table, counts, cap, hkv)


# ----------------------------------------------------------------------------- config 3 layer shape
def test_config3_layer_shape(gpu):
    """One layer at config 3's attention shape: the last 2048-token chunk of a 131072-token
    prompt (P = 2016 past blocks), 32 / 8 heads, about a quarter of the past kept.  Its 256 row
    tiles fill the CUs, so the plan runs unsplit (no partials, no merge); tables bit-exact,
    every attention row against the fp32 torch reference."""
    print("case: config 3 layer shape (chunk 2048 at the end of 131072 tokens, 32/8 heads)", flush=True)
    lq = 2048
    past = 131072 - lq
    ch = make_chunk_device(past, lq, HQ, HKV, gpu, seed=77)
    cap, P = ch.kv_cap, ch.past_blocks
    assert ops.attn_pick_splits(P, lq, HQ, HKV, cap) == 1
    kc, vc = torch.zeros_like(ch.k), torch.zeros_like(ch.v)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((HKV, cap, 128), dtype=torch.float32, device=gpu)
    _fill(ch, K, V, kmean, past, lq)
    qhat = ops.pool_query(ch.q, P, cap)
    topk, ratio = _calibrate(qhat, kmean, P, HKV, cap, lq // 64, 0.25)
    rowmask, table, counts = _select(qhat, kmean, P, HKV, cap, topk)
    _, _, sc = _oracle_scores(ch)
    _check_tables(rowmask, table, counts, sc, P, HKV, cap, topk)
    _check_attention(ch.q, kc, vc, P, table, counts, cap, HKV, oracle_rows=((lq - 2, lq),))


def test_config3_layer_attngate(gpu):
    """One layer at config 3's shape with config 3's selector: the last 2048-token chunk of a
    131072-token prompt (P = 2016 past blocks), 32 / 8 heads, AttnGate Qavg_Kavg with
    force_double (per-head 128 x 128 projections of the pooled Q and K ~ N(0, 0.02), block
    RoPE), softmax threshold 5e-3 + sink block + 2 local blocks.  Gate-K and gate-Q summaries,
    per-row masks, tables and counts bit-exact against the oracle; every attention row against
    the fp32 torch reference (the plan runs unsplit at this shape)."""
    from compactattention_amd.synthetic import rope_tables

    print("case: config 3 layer with AttnGate (chunk 2048 at the end of 131072 tokens, 32/8 heads)", flush=True)
    lq = 2048
    past = 131072 - lq
    ch = make_chunk_device(past, lq, HQ, HKV, gpu, seed=78)
    cap, P = ch.kv_cap, ch.past_blocks
    g = torch.Generator().manual_seed(1234)
    wq = (torch.randn((HQ, 128, 128), generator=g) * 0.02).float()
    wk = (torch.randn((HKV, 128, 128), generator=g) * 0.02).float()
    cos, sin = rope_tables(cap)
    kc, vc = torch.zeros_like(ch.k), torch.zeros_like(ch.v)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((HKV, cap, 128), dtype=torch.float32, device=gpu)
    kgate = torch.zeros_like(kmean)
    _fill(ch, K, V, kmean, past, lq, gate_wk=wk.to(gpu), rope_cos=cos.to(gpu), rope_sin=sin.to(gpu), kgate=kgate)
    rule = ops.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2)
    qhat = ops.pool_query(ch.q, P, cap, gate_wq=wq.to(gpu), rope_cos=cos.to(gpu), rope_sin=sin.to(gpu))
    rowmask, _ = ops.score_select(qhat, kgate, SCALE, rule, P, HKV, cap)
    table, counts, _, _ = ops.union_compact(rowmask, P, HKV, cap)
    torch.cuda.synchronize()
    nkb = P[0] + lq // 64
    means = oracle.block_mean(np.ascontiguousarray(bits(ch.k)[:, :, :nkb * 64].transpose(0, 2, 1, 3)))
    khat = np.zeros((1, HKV, cap, 128), dtype=np.float32)
    khat[:, :, :nkb] = oracle.gate_project(means, f32(wk), f32(cos), f32(sin), [0])
    assert float_bits_equal(f32(kgate[:, :nkb]).reshape(1, HKV, nkb, 128), khat[:, :, :nkb])
    qref = oracle.gate_project(oracle.block_mean(bits(ch.q)), f32(wq), f32(cos), f32(sin), P)
    assert float_bits_equal(f32(qhat), qref)
    keep = oracle.select_rows(oracle.block_scores(qref, khat, P, SCALE), P,
                              oracle.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2))
    assert np.array_equal(unpack_rowmask(rowmask, cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, HKV, P)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)
    assert ref_cnt.min() < nkb
    _check_attention(ch.q, kc, vc, P, table, counts, cap, HKV, oracle_rows=((lq - 2, lq),))


def test_config3_full_width_model(gpu):
    """Config 3's decoder at full width with two of its 32 layers: hidden 4096, 32 / 8 heads,
    SwiGLU 14336, vocab 128256, RoPE theta 5e5, random N(0, 0.02) bf16 weights, AttnGate
    Qavg_Kavg with force_double + threshold 5e-3 + sink + 2 local blocks at both layers; an
    8192-token prompt in 2048-token chunks (the first dense).  For each layer and each selecting
    chunk the tables the model built equal the oracle's, recomputed from the hidden states the
    layer received (gate pooling, projection, RoPE, scores, masks, unions), and the last
    chunk's attention rows match the fp32 torch reference over the layer's own K/V."""
    from compactattention_amd.chunked_prefill import synthetic_prompt
    from compactattention_amd.prefill_sparse.llama import SeerAttnLlamaChunkedDenseForCausalLM, SeerAttnLlamaConfig
    from compactattention_amd.prefill_sparse.llama.modeling_llama_common import apply_rotary_pos_emb, project_qkv
    from compactattention_amd.synthetic import BASELINE_SEER

    from .util import oracle_gate_summaries

    print("case: config 3 full-width model (2 layers, hidden 4096, 8192-token prompt, chunk 2048)", flush=True)
    tokens, chunk = 8192, 2048
    cfg = SeerAttnLlamaConfig(num_hidden_layers=2, max_position_embeddings=tokens, **BASELINE_SEER)
    model = SeerAttnLlamaChunkedDenseForCausalLM(cfg, device=gpu)
    model.init_weights(seed=1234)
    ids = synthetic_prompt(1, tokens, cfg.vocab_size, 1234 + 131072 * 104729, gpu)
    captured = {i: [] for i in range(2)}
    sinks = {}
    hooks = []
    for i, layer in enumerate(model.model.layers):
        attn = layer.self_attn
        attn.table_sink = sinks.setdefault(i, [])
        attn.compactattn_debug = True
        hooks.append(attn.register_forward_pre_hook(
            lambda mod, args, i=i: captured[i].append(args[0].detach().clone())))
    cache = model.new_cache(1, tokens)
    with torch.no_grad():
        for s0 in range(0, tokens, chunk):
            model(ids[:, s0:s0 + chunk], cache)
            # the tables of this chunk, per layer (the debug stats hold the last call's)
            for i, layer in enumerate(model.model.layers):
                st = layer.self_attn._compactattn_last_stats
                sinks[i][-1] = (st["table"].clone(), st["counts"].clone(), st["past_blocks"])
    for h in hooks:
        h.remove()
    bcos, bsin = (f32(t) for t in model.model.rotary_emb.blocks())
    rule = oracle.Rule(threshold=5e-3, sink_blocks=1, local_blocks=2)
    Hkv = cfg.num_key_value_heads
    for i, layer in enumerate(model.model.layers):
        attn = layer.self_attn
        with torch.no_grad():
            parts = [project_qkv(attn, h) for h in captured[i]]
        k_nope_all = torch.cat([p[1] for p in parts], dim=1)
        for c in range(1, tokens // chunk):  # chunk 0 is dense
            table, counts, past = sinks[i][c]
            P = [past]
            assert past == c * chunk // 64
            qhat, khat = oracle_gate_summaries(attn.attn_gate, bits(parts[c][0]), bits(k_nope_all[:, :(c + 1) * chunk]),
                                               bcos, bsin, P[0])
            keep = oracle.select_rows(oracle.block_scores(qhat, khat, P, 128 ** -0.5), P, rule)
            _, _, ref_tab, ref_cnt = oracle.union_compact(keep, Hkv, P)
            assert np.array_equal(counts.cpu().numpy(), ref_cnt), (i, c)
            assert np.array_equal(table.cpu().numpy()[:, :ref_tab.shape[1]], ref_tab), (i, c)
        # the last chunk's attention over the layer's own RoPE'd K/V
        cos, sin = model.model.rotary_emb.tokens(0, tokens)
        with torch.no_grad():
            q_last = parts[-1][0]
            k_all = torch.cat([p[1] for p in parts], dim=1)
            v_all = torch.cat([p[2] for p in parts], dim=1)
            qr, _ = apply_rotary_pos_emb(q_last, q_last, cos[-chunk:], sin[-chunk:])
            _, kr = apply_rotary_pos_emb(k_all, k_all, cos, sin)
        kc = kr.transpose(1, 2).contiguous()
        vc = v_all.transpose(1, 2).contiguous()
        table, counts, past = sinks[i][-1]
        out = ops.attn_fwd(qr.contiguous(), ops.KV.heads_first(kc), ops.KV.heads_first(vc), table, counts, [past],
                           SCALE, tokens // 64, Hkv)
        torch_reference_check(out, qr.contiguous(), kc, vc, [past], table, counts, SCALE)


# ----------------------------------------------------------------------------- config 4
def test_fullsize_config4_ragged(gpu):
    """Config 4: four requests with cached pasts 16384 / 49152 / 98304 / 131072 tokens, a
    512-token chunk each in one launch per kernel, 28 / 4 heads (G = 7), FlashPrefill pooled
    top-k 3 + sink block + 2 local blocks (about 20 % of the past blocks after the union)."""
    print("case: full-size config 4 (ragged batch, G = 7)", flush=True)
    pasts, lq, hq, hkv = (16384, 49152, 98304, 131072), 512, 28, 4
    B, qb = len(pasts), lq // 64
    P = [p // 64 for p in pasts]
    cap = max(P) + qb
    chs = [make_chunk_device(p, lq, hq, hkv, gpu, seed=1234 + i, kv_cap=cap) for i, p in enumerate(pasts)]
    q = torch.cat([c.q for c in chs], 0)
    k = torch.cat([c.k for c in chs], 0)  # [B, Hkv, cap*64, 128], zero past each request's end
    v = torch.cat([c.v for c in chs], 0)
    del chs
    kmean = torch.zeros((B * hkv, cap, 128), dtype=torch.float32, device=gpu)
    for b in range(B):
        ops.cache_fill(k[b:b + 1, :, :(P[b] + qb) * 64].transpose(1, 2).contiguous(), None, None, None, [0], cap,
                       kmean[b * hkv:(b + 1) * hkv])
    rule = ops.Rule(topk=3, sink_blocks=1, local_blocks=2)
    qhat = ops.pool_query(q, P, cap)
    rowmask, _ = ops.score_select(qhat, kmean, SCALE, rule, P, hkv, cap)
    table, counts, _, _ = ops.union_compact(rowmask, P, hkv, cap)
    torch.cuda.synchronize()
    kbits = bits(k)
    khat = np.zeros((B, hkv, cap, 128), dtype=np.float32)
    for b in range(B):
        n = P[b] + qb
        khat[b, :, :n] = oracle.block_mean(np.ascontiguousarray(kbits[b:b + 1, :, :n * 64].transpose(0, 2, 1, 3)))[0]
    assert float_bits_equal(f32(kmean).reshape(B, hkv, cap, 128), khat)
    qref = oracle.block_mean(bits(q))
    assert float_bits_equal(f32(qhat), qref)
    keep = oracle.select_rows(oracle.block_scores(qref, khat, P, SCALE), P,
                              oracle.Rule(topk=3, sink_blocks=1, local_blocks=2))
    assert np.array_equal(unpack_rowmask(rowmask, cap), keep)
    _, _, ref_tab, ref_cnt = oracle.union_compact(keep, hkv, P)
    assert np.array_equal(counts.cpu().numpy(), ref_cnt)
    assert np.array_equal(table.cpu().numpy(), ref_tab)
    kept = [float(((counts.cpu().view(B, hkv)[b] - qb).float() / P[b]).mean()) for b in range(B)]
    assert all(0.05 < r < 0.5 for r in kept), kept
    _check_attention(q, k, v, P, table, counts, cap, hkv, oracle_rows=((0, 2), (lq - 2, lq)))


# ------------------------------------------------------- one rank's share of 2-way sharding
@pytest.mark.parametrize("hkv", [4, 2, 6])
def test_sharded_share_fewer_rows_than_xcds(gpu, hkv):
    """One GPU's share of config 2 under KV-head sharding (2 and 4 ways: 4 / 16 and 2 / 8 KV /
    Q heads of a 131072-token cache) and a 6 / 24-head shape: KV rows that do not divide over
    the 8 XCDs, so the plan places single splits of each row on different XCDs.  Tables
    bit-exact against the oracle, every attention row against the fp32 torch reference, and
    the result equal to the unsplit plan within the same tolerance."""
    hq = hkv * HQ // HKV
    print(f"case: sharded share (131072 past tokens, chunk 1024, {hq}/{hkv} heads)", flush=True)
    ch = make_chunk_device(PAST, LQ, hq, hkv, gpu, seed=91)
    cap, P = ch.kv_cap, ch.past_blocks
    assert ops.attn_pick_splits(P, LQ, hq, hkv, cap) >= 8 // hkv
    kc, vc = torch.zeros_like(ch.k), torch.zeros_like(ch.v)
    K, V = ops.KV.heads_first(kc), ops.KV.heads_first(vc)
    kmean = torch.zeros((hkv, cap, 128), dtype=torch.float32, device=gpu)
    _fill(ch, K, V, kmean, PAST, LQ)
    qhat = ops.pool_query(ch.q, P, cap)
    rowmask, table, counts = _select(qhat, kmean, P, hkv, cap, TOPK)
    _, _, sc = _oracle_scores(ch)
    _check_tables(rowmask, table, counts, sc, P, hkv, cap, TOPK)
    out = _check_attention(ch.q, kc, vc, P, table, counts, cap, hkv, oracle_rows=((LQ - 2, LQ),))
    one = ops.attn_fwd(ch.q, K, V, table, counts, P, SCALE, cap, hkv, num_splits=1)
    err = (out.float() - one.float()).abs()
    assert err.max().item() <= ATOL_MAX and err.mean().item() <= ATOL_MEAN
