"""Pins the CPU oracle against independent restatements (CPU only).

Every oracle function is checked against something other than its own formula: fp64
numpy/torch evaluations of the reference's torch code paths, brute force on tiny inputs,
the reference's CSR spec for block tables, and closed-form special cases.  A mistake in
the oracle (a dropped term, a wrong index or sign, an off-by-one causal bound) fails one
of these.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle

from .util import ref_flashprefill_rowwise, ref_flashprefill_tables, ref_seer_tables

RNG = np.random.default_rng(1234)


def _bf16(shape, scale=1.0):
    x = (RNG.standard_normal(shape) * scale).astype(np.float32)
    return oracle.f32_to_bf16_bits(x)


def test_bf16_round_trip_and_rounding():
    x = np.array([1.0, -2.5, 3.14159, 1e-3, 65504.0, -0.0], np.float32)
    b = oracle.f32_to_bf16_bits(x)
    y = oracle.bf16_bits_to_f32(b)
    assert np.array_equal(y, torch.tensor(x).to(torch.bfloat16).float().numpy())


def test_exp_within_one_ulp():
    x = np.linspace(-80.0, 0.0, 400001, dtype=np.float32)
    e = oracle.exp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(e - ref) / ulp).max() <= 1.0
    assert oracle.exp(np.array([-81.0, -1000.0], np.float32)).tolist() == [0.0, 0.0]
    assert oracle.exp(np.array([0.0], np.float32))[0] == 1.0


def test_block_mean_matches_fp64():
    x = _bf16((2, 256, 3, 128))
    m = oracle.block_mean(x)
    ref = oracle.bf16_bits_to_f32(x).astype(np.float64).reshape(2, 4, 64, 3, 128).mean(axis=2).transpose(0, 2, 1, 3)
    assert m.shape == (2, 3, 4, 128)
    assert np.abs(m - ref).max() <= 1e-6


@pytest.mark.parametrize("L", [37, 64 * 3 + 5, 64 * 2 + 63])
def test_block_mean_partial_last_block(L):
    """A sequence of L tokens (not a multiple of 64) has ceil(L/64) blocks; the last averages
    only its L % 64 tokens (compute_mean_vector's sum over the valid tokens / their count,
    flashprefill_native_forward.py:78-88) -- an fp64 mean over those tokens; torch's
    avg_pool3d with ceil_mode (AttnGate's pooling, attn_gate.py:113-130) agrees, and max /
    min pooling covers those tokens only.  Whole blocks keep the 64-token mean bit for bit."""
    x = _bf16((2, L, 3, 128))
    nb = -(-L // 64)
    r = L - 64 * (nb - 1)
    m = oracle.block_mean(x)
    assert m.shape == (2, 3, nb, 128)
    xf = oracle.bf16_bits_to_f32(x).astype(np.float64)
    ref_last = xf[:, 64 * (nb - 1):].mean(axis=1)  # [B, H, D]
    assert np.abs(m[:, :, -1] - ref_last).max() <= 1e-6
    if nb > 1:
        assert float_bits_equal_np(m[:, :, :-1], oracle.block_mean(x[:, :64 * (nb - 1)]))
    got = oracle.block_pool(x, oracle.pool_bits(("max", "avg")))
    assert float_bits_equal_np(got[..., 128:], m)
    assert np.array_equal(got[:, :, -1, :128], xf[:, 64 * (nb - 1):].max(axis=1).astype(np.float32))
    if L >= 64:  # torch's pools refuse an input shorter than the kernel
        t = torch.from_numpy(oracle.bf16_bits_to_f32(x)).double()
        pooled = torch.nn.functional.avg_pool3d(t, kernel_size=[64, 1, 1], stride=[64, 1, 1], ceil_mode=True)
        assert np.abs(m - pooled.numpy().transpose(0, 2, 1, 3)).max() <= 1e-6
        mxp = torch.nn.functional.max_pool3d(t, kernel_size=[64, 1, 1], stride=[64, 1, 1], ceil_mode=True)
        assert np.array_equal(got[..., :128], mxp.numpy().transpose(0, 2, 1, 3).astype(np.float32))
    assert r < 64  # the case has a partial block


@pytest.mark.parametrize("L", [128 * 3, 128 * 3 + 64, 128 * 2 + 37, 128 * 2 + 64 + 37, 100])
def test_pair_block_means_are_128_token_means(L):
    """128-token summaries from the 64-token means equal the fp64 mean of each 128-token block's
    tokens (a partial last block's valid ones: compute_mean_vector at block_size 128,
    flashprefill_native_forward.py:78-88); whole pairs equal (m0 + m1) / 2 bit for bit."""
    x = _bf16((2, L, 3, 128))
    m64 = oracle.block_mean(x)  # [B, H, ceil(L/64), D]
    last = L - 64 * (m64.shape[2] - 1)
    m128 = oracle.pair_block_means(m64, last)
    nb = -(-L // 128)
    assert m128.shape == (2, 3, nb, 128)
    xf = oracle.bf16_bits_to_f32(x).astype(np.float64)
    for j in range(nb):
        ref = xf[:, 128 * j:min(L, 128 * j + 128)].mean(axis=1)
        assert np.abs(m128[:, :, j] - ref).max() <= 2e-6, j
    full = L // 128
    if full:
        half = ((m64[:, :, 0:2 * full:2] + m64[:, :, 1:2 * full:2]) * np.float32(0.5)).astype(np.float32)
        assert float_bits_equal_np(m128[:, :, :full], half)


def _rotate_half(x):
    x1, x2 = x[..., :64], x[..., 64:]
    return torch.cat((-x2, x1), dim=-1)


def test_gate_project_matches_reference_formula():
    """MultiHeadLinear einsum('bshi,hio->bsho') + apply_rotary_pos_emb (rotate_half) in fp64."""
    B, H, N = 2, 3, 5
    x = RNG.standard_normal((B, H, N, 128)).astype(np.float32)
    W = (RNG.standard_normal((H, 128, 128)) * 0.02).astype(np.float32)
    rows = 20
    inv = 1.0 / (500000.0 ** (np.arange(0, 128, 2) / 128.0))
    ang = (np.arange(rows) * 64)[:, None] * inv[None, :]
    emb = np.concatenate([ang, ang], axis=-1)
    cos, sin = np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)
    first = [3, 11]
    y = oracle.gate_project(x, W, cos, sin, first)
    xt = torch.tensor(x, dtype=torch.float64).permute(0, 2, 1, 3)  # [B, N, H, in]
    proj = torch.einsum("bshi,hio->bsho", xt, torch.tensor(W, dtype=torch.float64))
    pos = torch.tensor([[f + n for n in range(N)] for f in first])
    c = torch.tensor(cos, dtype=torch.float64)[pos].unsqueeze(2)
    s = torch.tensor(sin, dtype=torch.float64)[pos].unsqueeze(2)
    ref = (proj * c + _rotate_half(proj) * s).permute(0, 2, 1, 3).numpy()
    assert np.abs(y - ref).max() <= 1e-5
    # no RoPE tables: projection only
    y2 = oracle.gate_project(x, W, None, None, first)
    assert np.abs(y2 - proj.permute(0, 2, 1, 3).numpy()).max() <= 1e-5


def test_block_scores_causal_softmax():
    B, Hq, Hkv, Qb, cap = 2, 4, 2, 3, 11
    past = [5, 7]
    qhat = RNG.standard_normal((B, Hq, Qb, 128)).astype(np.float32) * 0.5
    khat = RNG.standard_normal((B, Hkv, cap, 128)).astype(np.float32) * 0.5
    s = oracle.block_scores(qhat, khat, past, 0.125)
    for b in range(B):
        for h in range(Hq):
            for q in range(Qb):
                n = past[b] + q + 1
                logit = khat[b, h // 2, :n].astype(np.float64) @ qhat[b, h, q].astype(np.float64) * 0.125
                p = np.exp(logit - logit.max())
                p /= p.sum()
                assert np.abs(s[b, h, q, :n] - p).max() <= 2e-6
                assert (s[b, h, q, n:] == 0).all()


def _ref_rowwise(scores, past, alpha, sink, window, causal_only_past_topk=0):
    """Restatement of _flashprefill_keep_block_from_scores_rowwise (flashprefill_prefill.py:
    596-666) with min_budget = 0, per row, in torch."""
    s = torch.tensor(scores, dtype=torch.float32)
    B, H, Qb, Kb = s.shape
    out = torch.zeros_like(s, dtype=torch.bool)
    for b in range(B):
        P = past[b]
        k_ids = torch.arange(Kb).view(1, 1, Kb)
        q_ids = torch.arange(P, P + Qb).view(1, Qb, 1)
        dist = q_ids - k_ids
        causal = dist >= 0
        row = s[b]
        finite = torch.isfinite(row) & causal
        row = torch.where(finite, row, torch.zeros_like(row))
        mx = row.max(dim=-1, keepdim=True).values
        keep = finite & (row >= mx * alpha)
        keep = (keep | (k_ids < sink) | (causal & (dist < window))) & causal
        out[b] = keep
    return out.numpy().astype(np.uint8)


def test_select_alpha_sink_window_matches_reference_rowwise():
    B, H, Qb, cap = 2, 3, 4, 40
    past = [20, 33]
    s = RNG.random((B, H, Qb, cap)).astype(np.float32)
    s[0, 1, 2, 5] = np.inf * -1
    s[1, 0, 0, 4] = np.nan
    got = oracle.select_rows(s, past, oracle.Rule(alpha=0.3, sink_blocks=2, window_blocks=4))
    assert np.array_equal(got, _ref_rowwise(s, past, 0.3, 2, 4))


def test_select_threshold_is_strict_and_causal():
    B, H, Qb, cap = 1, 2, 3, 16
    past = [10]
    s = np.full((B, H, Qb, cap), 0.01, np.float32)
    s[0, 0, 0, 3] = 0.02
    got = oracle.select_rows(s, past, oracle.Rule(threshold=0.01))
    assert got.sum() == 1 and got[0, 0, 0, 3] == 1
    got = oracle.select_rows(s, past, oracle.Rule(threshold=0.005))
    for q in range(Qb):
        n = past[0] + q + 1
        assert got[0, :, q, :n].all() and not got[0, :, q, n:].any()


def test_select_topk_brute_force_with_ties():
    B, H, Qb, cap = 2, 2, 3, 30
    past = [12, 25]
    s = (RNG.integers(0, 5, (B, H, Qb, cap)) * 0.25).astype(np.float32)  # many ties
    s[0, 0, 0, 2] = -0.0
    s[0, 0, 0, 3] = 0.0
    for k in (1, 4, 9, 100):
        got = oracle.select_rows(s, past, oracle.Rule(topk=k))
        for b in range(B):
            for h in range(H):
                for q in range(Qb):
                    cands = sorted(range(past[b]), key=lambda kb: (-float(s[b, h, q, kb]), kb))[:k]
                    ref = np.zeros(cap, np.uint8)
                    ref[cands] = 1
                    assert np.array_equal(got[b, h, q], ref), (k, b, h, q)


def test_select_min_budget_all_columns_matches_torch_topk():
    """The all-columns top-k (the reference's min_budget) against torch.topk on tie-free rows:
    continuous scores of both signs, no non-finite entries, so the only equal values are the
    zeroed non-causal columns, which the causal mask drops whichever of them topk picks.
    Negative scores put those zeros above causal entries (they use up budget) and make the
    last query block's row max negative (no zeroed column in that row)."""
    B, H, Qb = 2, 3, 4
    past = [9, 17]
    cap = max(past) + Qb + 3
    for signed in (False, True):
        s = RNG.standard_normal((B, H, Qb, cap)).astype(np.float32)
        if not signed:
            s = np.abs(s) + 0.01
        else:
            s[1, 2] = -np.abs(s[1, 2]) - 0.01  # all negative: a negative row max in the last block
        for k in (0, 1, 3, 8, 15, 40):
            for alpha in (0.0, 0.5, 1.5):
                rule = oracle.Rule(topk=k, topk_all_columns=True, alpha=alpha, sink_blocks=1, window_blocks=2)
                got = oracle.select_rows(s, past, rule)
                for b in range(B):
                    Kb = past[b] + Qb
                    for h in range(H):
                        ref = ref_flashprefill_rowwise(s[b, h, :, :Kb], past[b], alpha, 1, 2, k)
                        assert np.array_equal(got[b, h, :, :Kb], ref), (signed, k, alpha, b, h)
                        assert not got[b, h, :, Kb:].any()


def test_select_min_budget_all_columns_ties_and_nonfinite():
    """Ties (heavy), -0/+0, NaN and +-inf: the all-columns top-k equals a stable descending sort
    of the zeroed row (ties to the lower block id), and a brute-force ranking by (-value, id)."""
    B, H, Qb = 1, 2, 3
    past = [12]
    Kb = past[0] + Qb
    s = (RNG.integers(-2, 4, (B, H, Qb, Kb)) * 0.25).astype(np.float32)
    s[0, 0, 0, 2] = -0.0
    s[0, 0, 1, 5] = np.nan
    s[0, 1, 0, 7] = np.inf
    s[0, 1, 2, 3] = -np.inf
    for k in (1, 2, 5, 9, 14, 15, 30):
        rule = oracle.Rule(topk=k, topk_all_columns=True, alpha=0.25)
        got = oracle.select_rows(s, past, rule)
        for h in range(H):
            ref = ref_flashprefill_rowwise(s[0, h], past[0], 0.25, 0, 0, k, use_topk=False)
            assert np.array_equal(got[0, h], ref), (k, h)
            for q in range(Qb):
                n = past[0] + q + 1
                z = [float(s[0, h, q, kb]) if kb < n and np.isfinite(s[0, h, q, kb]) else 0.0 for kb in range(Kb)]
                picks = sorted(range(Kb), key=lambda kb: (-(z[kb] + 0.0), kb))[:k]
                for kb in picks:
                    if kb < n:
                        assert got[0, h, q, kb] == 1, (k, h, q, kb)


def test_select_past_only_topk_differs_from_all_columns():
    """The past-only top-k (this path's config-2 selector) spends the whole budget on past
    blocks; the all-columns form lets current-chunk blocks take part of it."""
    s = np.zeros((1, 1, 2, 12), np.float32)
    s[0, 0, :, :10] = np.linspace(0.1, 0.2, 10, dtype=np.float32)
    s[0, 0, :, 10:] = 1.0  # current-chunk blocks rank first
    past = [10]
    s[0, 0, 0, 11] = 0.0  # non-causal for query block 0
    a = oracle.select_rows(s, past, oracle.Rule(topk=3))
    b = oracle.select_rows(s, past, oracle.Rule(topk=3, topk_all_columns=True))
    assert a[0, 0, 1, :10].sum() == 3 and set(np.nonzero(a[0, 0, 1])[0]) == {7, 8, 9}
    assert set(np.nonzero(b[0, 0, 1])[0]) == {9, 10, 11}
    assert set(np.nonzero(b[0, 0, 0])[0]) == {8, 9, 10}


def test_select_local_blocks():
    s = np.zeros((1, 1, 2, 20), np.float32)
    got = oracle.select_rows(s, [10], oracle.Rule(local_blocks=2, sink_blocks=1))
    for q in range(2):
        assert set(np.nonzero(got[0, 0, q])[0].tolist()) == {0, 8, 9}


def _gate_like_scores(rng, B, H, Qb, cap, past):
    """Causal softmax rows (finite, summing to 1 over kb <= P + qb); the non-causal entries hold
    1.0 so that a rule reading them would keep them."""
    s = np.ones((B, H, Qb, cap), np.float32)
    for b in range(B):
        for q in range(Qb):
            n = past[b] + q + 1
            x = rng.standard_normal((H, n)) * 2.0
            e = np.exp(x - x.max(-1, keepdims=True))
            s[b, :, q, :n] = e / e.sum(-1, keepdims=True)
    return s


@pytest.mark.parametrize("Qb", [1, 3, 16])
@pytest.mark.parametrize("kv_group_aware", [False, True])
def test_seer_reference_rule_is_threshold_plus_local_blocks(Qb, kv_group_aware):
    """The reference's Seer selection (fast path + KV-head union, restated in torch in
    tests/util.ref_seer_tables) equals the oracle's strict threshold rule with local_blocks =
    max(0, keep_recent_blocks - Qb), Q-block union and GQA union: the mapping the operator entry
    and the Seer layer use.  Per-request thresholds select each request with its own value."""
    rng = np.random.default_rng(100 + Qb)
    Hkv, G = 2, 3
    past = [37, 90]
    cap = max(past) + Qb + 3
    H = Hkv if kv_group_aware else Hkv * G
    s = _gate_like_scores(rng, 2, H, Qb, cap, past)
    for keep_recent in (0, 1, 2, 4, Qb + 5, 200):
        for thr in (0.05, [0.02, 0.1]):
            ref_t, ref_c = ref_seer_tables(s, past, Hkv, thr, keep_recent, kv_group_aware=kv_group_aware)
            local = max(0, keep_recent - Qb)
            thrs = thr if isinstance(thr, list) else [thr, thr]
            keep = np.concatenate([oracle.select_rows(s[b:b + 1], past[b:b + 1],
                                                      oracle.Rule(threshold=thrs[b], local_blocks=local))
                                   for b in range(2)])
            _, _, t, c = oracle.union_compact(keep, Hkv, past)
            assert np.array_equal(c, ref_c), (keep_recent, thr)
            assert np.array_equal(t[:, :ref_t.shape[1]], ref_t), (keep_recent, thr)
            if keep_recent <= Qb + 1:
                assert (ref_c < np.repeat(np.array(past) + Qb, Hkv)).any(), "the case should drop blocks"


def test_union_compact_matches_reference_csr_spec():
    """Tables equal global_ids[keep_flat] - row*Kb of the reference's metadata spec
    (flashinfer_zero_copy_prefill.py:482-510) after the Q-block and GQA unions."""
    B, Hq, Hkv, Qb, cap = 2, 6, 2, 4, 30
    past = [10, 26]
    rowkeep = (RNG.random((B, Hq, Qb, cap)) < 0.15).astype(np.uint8)
    for last_n in (0, 2):
        kbk, kv, tab, cnt = oracle.union_compact(rowkeep, Hkv, past, last_n)
        pooled = Qb - min(last_n, Qb - 1)
        for b in range(B):
            P, nkb = past[b], past[b] + Qb
            ref_kb = rowkeep[b, :, :pooled, :].any(axis=1)
            ref_kb[:, P:nkb] = True
            ref_kb[:, nkb:] = False
            assert np.array_equal(kbk[b], ref_kb.astype(np.uint8))
            ref_kv = ref_kb.reshape(Hkv, Hq // Hkv, cap).any(axis=1)
            assert np.array_equal(kv[b], ref_kv.astype(np.uint8))
        keep_flat = torch.tensor(kv.reshape(B * Hkv, cap).astype(bool))
        global_ids = torch.arange(B * Hkv * cap).view(B * Hkv, cap)
        kv_indices = global_ids[keep_flat]
        indptr = torch.zeros(B * Hkv + 1, dtype=torch.long)
        indptr[1:] = keep_flat.sum(1).cumsum(0)
        for r in range(B * Hkv):
            ids = (kv_indices[indptr[r]:indptr[r + 1]] - r * cap).numpy()
            assert cnt[r] == len(ids)
            assert np.array_equal(tab[r, :cnt[r]], ids)
            assert (tab[r, cnt[r]:] == -1).all()


def test_union_g1_identity_and_idempotent():
    B, H, Qb, cap = 1, 3, 2, 12
    past = [8]
    rowkeep = (RNG.random((B, H, Qb, cap)) < 0.3).astype(np.uint8)
    kbk, kv, tab, cnt = oracle.union_compact(rowkeep, H, past)
    assert np.array_equal(kbk, kv)
    # feeding the union back as rows changes nothing
    again = np.repeat(kbk[:, :, None, :], Qb, axis=2)
    kbk2, kv2, tab2, cnt2 = oracle.union_compact(again, H, past)
    assert np.array_equal(kv2, kv) and np.array_equal(tab2, tab) and np.array_equal(cnt2, cnt)


def _sdpa_ref(qf, kf, vf, past_tok, keys_sel, scale):
    """fp64 softmax(q k^T) v with an explicit key mask (selected keys & causal)."""
    Lq = qf.shape[0]
    s = (qf @ kf.T) * scale
    pos = past_tok + np.arange(Lq)
    mask = keys_sel[None, :] & (np.arange(kf.shape[0])[None, :] <= pos[:, None])
    s = np.where(mask, s, -np.inf)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    return (p / p.sum(axis=1, keepdims=True)) @ vf


def test_attention_matches_masked_sdpa_and_dense():
    B, Lq, Hq, Hkv, cap = 1, 64, 4, 2, 6
    past = [4]
    q = _bf16((B, Lq, Hq, 128))
    k = _bf16((B, Hkv, cap * 64, 128))
    v = _bf16((B, Hkv, cap * 64, 128))
    table = np.full((Hkv, cap), -1, np.int32)
    table[0, :3] = [1, 3, 4]
    table[1, :2] = [0, 4]
    table[1, 2] = 5
    table[0, 3] = 5
    counts = np.array([4, 3], np.int32)
    out = oracle.attention(q, k, v, past, table, counts, 0.1)
    qf, kf, vf = (oracle.bf16_bits_to_f32(a).astype(np.float64) for a in (q, k, v))
    for h in range(Hq):
        hk = h // 2
        sel = np.zeros(cap * 64, bool)
        for blk in table[hk, :counts[hk]]:
            sel[blk * 64:(blk + 1) * 64] = True
        ref = _sdpa_ref(qf[0, :, h], kf[0, hk], vf[0, hk], past[0] * 64, sel, 0.1)
        assert np.abs(out[0, :, h] - ref).max() <= 1e-6
    # all blocks selected == dense causal attention (torch SDPA in fp64)
    dense_tab = np.tile(np.arange(cap, dtype=np.int32), (Hkv, 1))
    out_d = oracle.attention(q, k, v, past, dense_tab, np.full(Hkv, cap, np.int32), 0.1)
    qt = torch.tensor(qf).permute(0, 2, 1, 3)
    kt = torch.tensor(kf).repeat_interleave(2, dim=1)
    vt = torch.tensor(vf).repeat_interleave(2, dim=1)
    mask = torch.arange(cap * 64)[None, :] <= (past[0] * 64 + torch.arange(Lq))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=0.1)
    assert np.abs(out_d - ref.permute(0, 2, 1, 3).numpy()).max() <= 1e-6


def test_attention_decode_pins():
    """Decode (q_len newest tokens over the whole cache, bottom-right causal mask): pinned to
    torch's lower-right causal SDPA (fp64, ragged and unaligned lengths), to the C oracle's
    prefill attention on 64-aligned shapes, and to the one-key closed form."""
    from torch.nn.attention.bias import causal_lower_right

    B, Hq, Hkv, Lq = 3, 6, 2, 5
    kv_len = [5, 77, 200]
    q = _bf16((B, Lq, Hq, 128))
    k = _bf16((B, Hkv, 256, 128))
    v = _bf16((B, Hkv, 256, 128))
    nan = oracle.f32_to_bf16_bits(np.array([np.nan], np.float32))[0]
    for b, n in enumerate(kv_len):  # tokens past kv_len are never read
        k[b, :, n:] = nan
        v[b, :, n:] = nan
    out, lse = oracle.attention_decode(q, k, v, kv_len, 0.09, with_lse=True)
    assert np.isfinite(out).all() and np.isfinite(lse).all()
    qf, kf, vf = (oracle.bf16_bits_to_f32(a).astype(np.float64) for a in (q, k, v))
    for b, n in enumerate(kv_len):
        qt = torch.tensor(qf[b]).permute(1, 0, 2)[None]  # [1, Hq, Lq, D]
        kt = torch.tensor(kf[b, :, :n]).repeat_interleave(Hq // Hkv, dim=0)[None]
        vt = torch.tensor(vf[b, :, :n]).repeat_interleave(Hq // Hkv, dim=0)[None]
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=causal_lower_right(Lq, n),
                                                               scale=0.09)
        assert np.abs(out[b] - ref[0].permute(1, 0, 2).numpy()).max() <= 1e-6
        s = torch.einsum("hqd,hkd->hqk", qt[0], kt[0]) * 0.09
        s = s.masked_fill(torch.arange(n)[None, :] > (n - Lq + torch.arange(Lq))[:, None], float("-inf"))
        assert np.abs(lse[b] - torch.logsumexp(s, dim=-1).numpy()).max() <= 1e-5

    # 64-aligned shapes: decode over kv_len = 64 (P + 1) equals prefill of the last block
    past = [3, 0]
    Lq = 64
    cap = 4
    q = _bf16((2, Lq, Hq, 128))
    k = _bf16((2, Hkv, cap * 64, 128))
    v = _bf16((2, Hkv, cap * 64, 128))
    dense_tab = np.tile(np.arange(cap, dtype=np.int32), (2 * Hkv, 1))
    counts = np.array([4, 4, 1, 1], np.int32)
    pre, pre_lse = oracle.attention(q, k, v, past, dense_tab, counts, 0.1, with_lse=True)
    dec, dec_lse = oracle.attention_decode(q, k, v, [64 * (p + 1) for p in past], 0.1, with_lse=True)
    assert np.abs(pre - dec).max() <= 1e-6
    assert np.abs(pre_lse - dec_lse).max() <= 1e-5

    # one key: the output is that key's value row and the log-sum-exp its score
    q1, k1, v1 = _bf16((1, 1, 2, 128)), _bf16((1, 1, 64, 128)), _bf16((1, 1, 64, 128))
    o1, l1 = oracle.attention_decode(q1, k1, v1, [1], 0.3, with_lse=True)
    vv = oracle.bf16_bits_to_f32(v1[0, 0, 0])
    assert np.array_equal(o1[0, 0, 0], vv) and np.array_equal(o1[0, 0, 1], vv)
    qq, kk = (oracle.bf16_bits_to_f32(a).astype(np.float64) for a in (q1[0, 0], k1[0, 0, 0]))
    assert np.abs(l1[0, :, 0] - 0.3 * (qq @ kk)).max() <= 1e-5


def test_planted_blocks_recalled_on_config0_shape():
    """Config 0: 256 queries over 8192 KV (P=124, C=4), 32/8 heads, FlashPrefill pooled scores,
    top-k + sink 0 + 2 local blocks at about 25 % post-union keep: the planted blocks are
    kept far above chance."""
    from compactattention_amd.synthetic import make_chunk

    ch = make_chunk([8192 - 256], 256, 32, 8, seed=1234)
    P = ch.past_blocks
    khat = oracle.block_mean(np.ascontiguousarray(
        ch.k.transpose(1, 2).contiguous().view(torch.int16).numpy().view(np.uint16)))
    qhat = oracle.block_mean(ch.q.view(torch.int16).numpy().view(np.uint16))
    sc = oracle.block_scores(qhat, khat, P, 1 / math.sqrt(128))
    best = None
    for k in range(1, 40):
        keep = oracle.select_rows(sc, P, oracle.Rule(topk=k, sink_blocks=1, local_blocks=2))
        _, kv, _, cnt = oracle.union_compact(keep, 8, P)
        ratio = (cnt - 4).mean() / P[0]
        if best is None or abs(ratio - 0.25) < abs(best[0] - 0.25):
            best = (ratio, kv)
    ratio, kv = best
    assert 0.2 <= ratio <= 0.3
    planted = ch.planted[0]
    hits = sum(int(kv[0, h, blk]) for h in range(8) for blk in planted[h])
    recall = hits / sum(len(p) for p in planted)
    assert recall >= 0.5, recall


def test_oracle_flashprefill_path_matches_reference_tables():
    """Oracle selection + union with the all-columns top-k (and last_n_block) equals the
    reference restatement's per-KV-group tables on continuous scores."""
    B, Hq, Hkv, Qb = 2, 6, 2, 4
    past = [11, 23]
    cap = max(past) + Qb + 2
    s = RNG.random((B, Hq, Qb, cap)).astype(np.float32) + 1e-3
    for k, last_n in ((0, 0), (3, 1), (9, 2), (40, 0)):
        rule = oracle.Rule(topk=k, topk_all_columns=True, alpha=0.4, sink_blocks=1, window_blocks=2, last_n_block=last_n)
        _, _, tab, cnt = oracle.union_compact(oracle.select_rows(s, past, rule), Hkv, past, last_n)
        rtab, rcnt = ref_flashprefill_tables(s, past, Hkv, 0.4, 1, 2, k, last_n)
        assert np.array_equal(cnt, rcnt) and np.array_equal(tab, rtab), (k, last_n)


def test_block_pool_matches_numpy():
    """max / min pooling equal numpy's over the bf16 values exactly; avg equals block_mean;
    the pools are concatenated max, min, avg (the reference's torch.cat order over
    combinations of ('max', 'min', 'avg'), attn_gate.py:124-130,265-278)."""
    x = _bf16((2, 192, 3, 128))
    xf = oracle.bf16_bits_to_f32(x).reshape(2, 3, 64, 3, 128)  # [B, nb, 64, H, D]
    mx = xf.max(axis=2).transpose(0, 2, 1, 3)
    mn = xf.min(axis=2).transpose(0, 2, 1, 3)
    avg = oracle.block_mean(x)
    for names in (("max",), ("min",), ("avg",), ("max", "avg"), ("min", "avg"), ("max", "min", "avg")):
        got = oracle.block_pool(x, oracle.pool_bits(names))
        ref = np.concatenate([{"max": mx, "min": mn, "avg": avg}[n] for n in names], axis=-1)
        assert got.shape == (2, 3, 3, 128 * len(names))
        assert float_bits_equal_np(got, ref), names


def float_bits_equal_np(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


def test_gate_project_wide_input_matches_multiheadlinear():
    """Projection of C*128 (and G*C*128) pooled inputs against the reference's MultiHeadLinear
    einsum in fp64, including its repeat of K heads to the Q heads (repeat_kv_varlen,
    modules/common.py:186-193) and the kv-group-aware query reshape (attn_gate.py:96-111)."""
    B, Hkv, G, N = 1, 2, 3, 4
    Hq = Hkv * G
    C = 3
    kp = RNG.standard_normal((B, Hkv, N, C * 128)).astype(np.float32)
    Wk = (RNG.standard_normal((Hq, C * 128, 128)) * 0.02).astype(np.float32)
    # K repeated to the Q heads (head hk*G + j uses KV head hk), projected per Q head
    rep = np.repeat(kp, G, axis=1)
    got = oracle.gate_project(rep, Wk, None, None, [0])
    x = torch.tensor(kp, dtype=torch.float64).permute(0, 2, 1, 3)  # [B, N, Hkv, in]
    xr = x.unsqueeze(-2).expand(B, N, Hkv, G, C * 128).reshape(B, N, Hq, C * 128)
    ref = torch.einsum("bshi,hio->bsho", xr, torch.tensor(Wk, dtype=torch.float64)).permute(0, 2, 1, 3)
    assert np.abs(got - ref.numpy()).max() <= 1e-5
    # kv-group-aware query: the G heads' pooled vectors of a group concatenated head-major
    qp = RNG.standard_normal((B, Hq, N, 128)).astype(np.float32)
    Wq = (RNG.standard_normal((Hkv, G * 128, 128)) * 0.02).astype(np.float32)
    cat = qp.reshape(B, Hkv, G, N, 128).transpose(0, 1, 3, 2, 4).reshape(B, Hkv, N, G * 128)
    got = oracle.gate_project(cat, Wq, None, None, [0])
    q = torch.tensor(qp, dtype=torch.float64).permute(0, 2, 1, 3)  # [B, N, Hq, 128]
    grouped = q.contiguous().view(B, N, Hkv, G, 128).reshape(B, N, Hkv, G * 128)
    ref = torch.einsum("bshi,hio->bsho", grouped, torch.tensor(Wq, dtype=torch.float64)).permute(0, 2, 1, 3)
    assert np.abs(got - ref.numpy()).max() <= 1e-5


def test_torch_restatement_matches_oracle():
    """The fp32 torch restatement timed as the CPU baseline (oracle/torch_ref.py) selects the
    oracle's tables and attends within fp32 rounding of the fp64 oracle."""
    from compactattention_amd.synthetic import make_chunk
    from oracle import torch_ref

    Hq, Hkv, Lq, past = 8, 2, 128, 64 * 12
    ch = make_chunk([past], Lq, Hq, Hkv, seed=21)
    P = ch.past_blocks[0]
    k, v = ch.k.float(), ch.v.float()  # [1, Hkv, cap*64, D]
    k_new = k[:, :, past:past + Lq].transpose(1, 2)
    v_new = v[:, :, past:past + Lq].transpose(1, 2)
    kmean_past = torch_ref.block_means(k[:, :, :past].transpose(1, 2))
    out, k_all, v_all, _, tables = torch_ref.chunk_step(ch.q.float(), k[:, :, :past], v[:, :, :past], k_new, v_new,
                                                         kmean_past, topk=3)
    qb = ch.q.view(torch.int16).numpy().view(np.uint16)
    kb = ch.k.view(torch.int16).numpy().view(np.uint16)
    vb = ch.v.view(torch.int16).numpy().view(np.uint16)
    khat = oracle.block_mean(np.ascontiguousarray(kb.transpose(0, 2, 1, 3)))
    sc = oracle.block_scores(oracle.block_mean(qb), khat, [P], 1 / math.sqrt(128))
    keep = oracle.select_rows(sc, [P], oracle.Rule(topk=3, sink_blocks=1, local_blocks=2))
    _, _, tab, cnt = oracle.union_compact(keep, Hkv, [P])
    for r in range(Hkv):
        assert tables[r].tolist() == tab[r, :cnt[r]].tolist()
    ref = oracle.attention(qb, kb, vb, [P], tab, cnt, 1 / math.sqrt(128))
    assert np.abs(out.numpy() - ref).max() <= 1e-4


def test_torch_restatement_rope_and_layer():
    """The CPU decoder layer timed for the config-3 extrapolation (oracle/torch_ref.py):
    - rope rotates each (x_i, x_{i+64}) pair by pos * theta^(-2i/128), checked element by
      element in fp64;
    - decoder_layer_step with every past block kept equals a dense layer written here with
      torch SDPA (pre-norm residual blocks, SwiGLU), so norm placement, residuals and the
      projection layout are pinned; a planted mistake (the MLP without its RMSNorm) fails."""
    from oracle import torch_ref

    g = torch.Generator().manual_seed(3)
    x = torch.randn((1, 6, 2, 128), generator=g)
    pos = torch.arange(6) + 1000
    y = torch_ref.rope(x, pos).double()
    inv = 1.0 / (500000.0 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    ang = pos.double()[:, None] * inv[None, :]  # [L, 64]
    c, s = ang.cos()[None, :, None, :], ang.sin()[None, :, None, :]
    xd = x.double()
    ref = torch.cat([xd[..., :64] * c - xd[..., 64:] * s, xd[..., 64:] * c + xd[..., :64] * s], dim=-1)
    assert torch.allclose(y, ref, atol=1e-5)

    hid, hq, hkv, inter, L, past = 256, 4, 2, 384, 64, 128
    D = 128

    def W(o, i):
        return torch.randn((o, i), generator=g) * 0.05

    w = {"ln1": 1 + 0.1 * torch.randn(hid, generator=g), "wq": W(hq * D, hid), "wk": W(hkv * D, hid),
         "wv": W(hkv * D, hid), "wo": W(hid, hq * D), "ln2": 1 + 0.1 * torch.randn(hid, generator=g),
         "wg": W(inter, hid), "wu": W(inter, hid), "wd": W(hid, inter)}
    h = torch.randn((1, L, hid), generator=g)
    k_past = torch.randn((1, hkv, past, D), generator=g)
    v_past = torch.randn((1, hkv, past, D), generator=g)
    kmean_past = torch_ref.block_means(k_past.transpose(1, 2))
    got = torch_ref.decoder_layer_step(h, w, k_past, v_past, kmean_past, hq, hkv, topk=past // 64)

    def dense_layer(mlp_norm=True):
        p = torch.arange(L) + past
        x = torch_ref.rms_norm(h, w["ln1"])
        q = torch_ref.rope((x @ w["wq"].T).view(1, L, hq, D), p).transpose(1, 2)
        k = torch_ref.rope((x @ w["wk"].T).view(1, L, hkv, D), p).transpose(1, 2)
        v = (x @ w["wv"].T).view(1, L, hkv, D).transpose(1, 2)
        k = torch.cat([k_past, k], dim=2).repeat_interleave(hq // hkv, dim=1)
        v = torch.cat([v_past, v], dim=2).repeat_interleave(hq // hkv, dim=1)
        mask = torch.arange(past + L)[None, :] <= (past + torch.arange(L))[:, None]
        a = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask)
        hh = h + a.transpose(1, 2).reshape(1, L, hq * D) @ w["wo"].T
        x = torch_ref.rms_norm(hh, w["ln2"]) if mlp_norm else hh
        return hh + (torch.nn.functional.silu(x @ w["wg"].T) * (x @ w["wu"].T)) @ w["wd"].T

    assert torch.allclose(got, dense_layer(), atol=1e-4, rtol=1e-4)
    assert not torch.allclose(got, dense_layer(mlp_norm=False), atol=1e-3, rtol=1e-3)
