"""Pins of the oracle's FlashPrefill per-token scores (oracle.token_mass_scores), on the CPU.

The oracle restates compute_block_score_chunked + normalize_scores
(compact_attn/flashprefill_vendor/flashprefill_native_forward.py:98-207,365-374) with the
max shift of the reference.  Checked here against:
  - the closed form without the shift, written independently with torch in fp64:
    score[kb] = sum_t [t sees kb] 2^(s[t,kb]) / sum_kb' sum_t [t sees kb'] 2^(s[t,kb']),
    where slot t of query block qb sees key block kb iff start + BS qb + t >= BS kb + BS - 1;
  - zero queries, where every seen (slot, block) pair weighs 1: the score is the count of
    slots that see the block over the row's total count;
  - a planted mistake (the causal edge at the key block's first token instead of its last)
    that the closed form rejects.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

LOG2E = 1.4426950408889634


def _inputs(B, Lq, Hq, Hkv, nk_max, seed, spread=0.5):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn((B, Lq, Hq, 128), generator=g) * spread).to(torch.bfloat16)
    k = torch.randn((B, Hkv, nk_max, 128), generator=g) * spread
    return q.view(torch.int16).numpy().view(np.uint16), k.numpy().astype(np.float32), q, k


def _closed_form(q, k, past, scale, bs, cap, edge_offset=None):
    """fp64 closed form with torch (no max shift); edge_offset replaces BS - 1 in the causal
    edge (for the planted mistake)."""
    q = q.to(torch.float64)
    k = k.to(torch.bfloat16).to(torch.float64)  # the reference's bf16 mean_k
    B, Lq, Hq, _ = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    Qb = -(-Lq // bs)
    edge = bs - 1 if edge_offset is None else edge_offset
    out = torch.zeros((B, Hq, Qb, cap), dtype=torch.float64)
    for b in range(B):
        P = past[b]
        nk = P + Qb
        for h in range(Hq):
            for qb in range(Qb):
                slots = torch.zeros((bs, 128), dtype=torch.float64)
                n = min(bs, Lq - qb * bs)
                slots[:n] = q[b, qb * bs:qb * bs + n, h]
                qmax = P * bs + qb * bs + bs - 1
                hi = min(-(-(qmax + 1) // bs), nk)
                pos = P * bs + qb * bs + torch.arange(bs, dtype=torch.float64)
                kb = torch.arange(hi, dtype=torch.float64)
                sees = pos[:, None] >= (kb * bs + edge)[None, :]
                s = slots @ k[b, h // G, :hi].T * scale * LOG2E
                w = torch.where(sees, torch.exp2(s), torch.zeros_like(s)).sum(0)
                out[b, h, qb, :hi] = w / w.sum()
    return out.numpy()


@pytest.mark.parametrize("bs,Lq,past,G", [(64, 256, [7], 1), (64, 192 + 13, [3, 9], 2), (128, 384, [4], 4),
                                          (128, 128 + 50, [2, 0], 2)])
def test_token_mass_oracle_matches_closed_form(bs, Lq, past, G):
    B, Hkv = len(past), 2
    Hq = Hkv * G
    Qb = -(-Lq // bs)
    cap = max(past) + Qb + 1
    q_bits, k, q, kt = _inputs(B, Lq, Hq, Hkv, cap, seed=bs + Lq + G)
    scale = 128 ** -0.5
    got = oracle.token_mass_scores(q_bits, k, past, scale, bs, cap)
    ref = _closed_form(q, kt, past, scale, bs, cap)
    assert np.allclose(got, ref, rtol=1e-8, atol=1e-12)  # the reference's +1e-9 in the denominator
    # a planted mistake: the causal edge at the key block's first token
    bad = _closed_form(q, kt, past, scale, bs, cap, edge_offset=0)
    assert not np.allclose(got, bad, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("bs", [64, 128])
def test_token_mass_oracle_zero_queries_count_slots(bs):
    """Zero queries: s = 0 wherever a slot sees a block, so the score is the fraction of the
    row's (slot, block) pairs that fall on the block (slots past q_len count too, as in the
    reference)."""
    B, Lq, Hq, Hkv, past = 1, bs + 20, 2, 1, [5]
    Qb = -(-Lq // bs)
    cap = past[0] + Qb
    q_bits = np.zeros((B, Lq, Hq, 128), dtype=np.uint16)
    k = np.random.default_rng(0).standard_normal((B, Hkv, cap, 128)).astype(np.float32)
    got = oracle.token_mass_scores(q_bits, k, past, 0.1, bs, cap)
    for qb in range(Qb):
        pos = past[0] * bs + qb * bs + np.arange(bs)
        qmax = past[0] * bs + qb * bs + bs - 1
        hi = min(-(-(qmax + 1) // bs), cap)
        counts = np.array([(pos >= kb * bs + bs - 1).sum() for kb in range(hi)], dtype=np.float64)
        expect = np.zeros(cap)
        expect[:hi] = counts / counts.sum()
        assert np.allclose(got[0, 0, qb], expect, rtol=1e-8, atol=1e-12), qb
        # past blocks are seen by every slot
        assert np.all(counts[:past[0]] == bs)
