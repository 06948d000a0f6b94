"""Shared helpers for the parity tests (conversion between torch and the oracle's arrays)."""
from __future__ import annotations

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns (host numpy)."""
    assert t.dtype == torch.bfloat16
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().contiguous().numpy()


def unpack_rowmask(rowmask: torch.Tensor, cap: int) -> np.ndarray:
    """[..., words] int32 bitmask -> [..., cap] uint8 (bit kb%32 of word kb/32)."""
    w = rowmask.detach().cpu().numpy().view(np.uint32)
    bitsarr = (w[..., :, None] >> np.arange(32, dtype=np.uint32)) & 1
    flat = bitsarr.reshape(*w.shape[:-1], w.shape[-1] * 32)
    return flat[..., :cap].astype(np.uint8)


def float_bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


def pack_rowmask(keep: np.ndarray, cap: int) -> np.ndarray:
    """[..., cap] 0/1 -> [..., words] uint32 bitmask (inverse of unpack_rowmask)."""
    words = (cap + 31) // 32
    padded = np.zeros(keep.shape[:-1] + (words * 32,), np.uint64)
    padded[..., :cap] = keep
    w = (padded.reshape(keep.shape[:-1] + (words, 32)) << np.arange(32, dtype=np.uint64)).sum(-1)
    return w.astype(np.uint32)


def ref_flashprefill_rowwise(scores_row, P, alpha, sink, window, min_budget, use_topk=True):
    """Restatement of _flashprefill_keep_block_from_scores_rowwise (compact_attn/modules/
    flashprefill_prefill.py:596-666) for one (request, Q head) slice of Kb = P + Qb columns:
    the zeroed row (non-causal and non-finite entries 0), the alpha rule against the max of
    that row, min_budget by torch.topk over all Kb columns, sink, window, causal mask.
    Returns the per-query-block keep rows [Qb, Kb] (0/1).  With use_topk=False the top-k is
    a stable descending sort (ties to the lower block id) instead of torch.topk."""
    s = torch.as_tensor(np.asarray(scores_row), dtype=torch.float32)  # [Qb, Kb]
    Qb, Kb = s.shape
    k_ids = torch.arange(Kb).view(1, Kb)
    q_ids = torch.arange(P, P + Qb).view(Qb, 1)
    dist = q_ids - k_ids
    causal = dist >= 0
    finite = torch.isfinite(s) & causal
    row = torch.where(finite, s, torch.zeros_like(s))
    if min_budget > 0:
        k = min(int(min_budget), Kb)
        if use_topk:
            vals, idx = torch.topk(row, k=k, dim=-1)
        else:
            vals, idx = torch.sort(row, dim=-1, descending=True, stable=True)
            vals, idx = vals[:, :k], idx[:, :k]
        mx = vals[:, :1]
        keep = finite & (row >= mx * alpha)
        keep.scatter_(-1, idx, True)
    else:
        mx = row.max(dim=-1, keepdim=True).values
        keep = finite & (row >= mx * alpha)
    keep = (keep | (k_ids < sink) | (causal & (dist < window))) & causal
    return keep.numpy().astype(np.uint8)


def ref_flashprefill_tables(scores, past, Hkv, alpha, sink, window, min_budget, last_n_block):
    """Per-KV-group block tables from [B, Hq, Qb, >= P+Qb] scores through the reference's
    rowwise rule (ref_flashprefill_rowwise), its Q-block union over the first
    Qb - last_n_block query blocks (:609-610,648), current blocks kept, the GQA union
    (:656-665) and ascending compaction.  Returns (table [B*Hkv, cap] -1 padded, counts)."""
    B, Hq, Qb, cap = scores.shape
    G = Hq // Hkv
    tail = min(max(last_n_block, 0), Qb - 1) if Qb > 1 else 0
    pooled = max(Qb - tail, 1)
    table = np.full((B * Hkv, cap), -1, np.int32)
    counts = np.zeros((B * Hkv,), np.int32)
    for b in range(B):
        P = int(past[b])
        Kb = P + Qb
        kq = np.zeros((Hq, Kb), bool)
        for h in range(Hq):
            rows = ref_flashprefill_rowwise(scores[b, h, :pooled, :Kb], P, alpha, sink, window, min_budget)
            kq[h] = rows.any(axis=0)
        kq[:, P:] = True
        kv = kq.reshape(Hkv, G, Kb).any(axis=1)
        for hk in range(Hkv):
            ids = np.nonzero(kv[hk])[0]
            table[b * Hkv + hk, :len(ids)] = ids
            counts[b * Hkv + hk] = len(ids)
    return table, counts


def oracle_gate_summaries(gate, q_bits, k_bits, cos, sin, q_first_block):
    """The oracle's (qhat, khat) for an AttnGate of any type: pooling by the gate's pool sets,
    then the reference's projection case (attn_gate.py:74-86) -- no query projection (the K
    blocks repeated to the Q heads and projected per Q head), per-Q-head projections, or the
    kv-group-aware query over the group's concatenated pooled heads -- and block RoPE.
    q_bits [B, Lq, Hq, 128], k_bits [B, K, Hkv, 128] (K blocks from block 0); cos/sin fp32
    [rows, 128] numpy tables by absolute block id."""
    import oracle

    B, _, Hq, _ = q_bits.shape
    Hkv = k_bits.shape[2]
    G = Hq // Hkv
    qp = oracle.block_pool(q_bits, oracle.pool_bits(gate.q_pooling_funcs))
    kp = oracle.block_pool(k_bits, oracle.pool_bits(gate.k_pooling_funcs))
    first = [q_first_block] * B
    wk = gate.mask_linear_k.weight.detach().float().cpu().numpy()
    if gate.mask_linear_q is None:
        eye = np.tile(np.eye(128, dtype=np.float32), (Hq, 1, 1))
        qhat = oracle.gate_project(qp, eye, cos, sin, first)
        kp = np.repeat(kp, G, axis=1)
    else:
        wq = gate.mask_linear_q.weight.detach().float().cpu().numpy()
        if gate.kv_group_aware_query:
            Qb, w = qp.shape[2], qp.shape[3]
            qp = qp.reshape(B, Hkv, G, Qb, w).transpose(0, 1, 3, 2, 4).reshape(B, Hkv, Qb, G * w)
        qhat = oracle.gate_project(qp, wq, cos, sin, first)
    khat = oracle.gate_project(kp, wk, cos, sin, [0] * B)
    return qhat, khat


def torch_reference_check(out, q, k_hf, v_hf, past_blocks, table, counts, scale, lse=None, atol_max=2e-2,
                          atol_mean=2e-3, lse_atol=4e-3):
    """Every query row of ``out`` ([B, Lq, Hq, 128] bf16, on the GPU) against an fp32 torch
    attention on the GPU over the blocks its KV row's table lists: gather those 64-token blocks
    of K and V, s = q k^T * scale where key position <= query position (the chunk's token t
    sits at 64 * past_blocks[b] + t), softmax, times V.  An independent reference (torch's
    fp32 GEMMs and softmax, no code shared with the kernel or the C oracle).  Checks the
    north-star tolerance over all rows and, if given, the log-sum-exp ``lse`` [B, Hq, Lq].
    Returns (max-abs, mean-abs)."""
    B, Lq, Hq, D = q.shape
    Hkv = k_hf.shape[1]
    G = Hq // Hkv
    dev = q.device
    tab = table.detach().cpu()
    cnt = counts.detach().cpu()
    worst, total, n = 0.0, 0.0, 0
    lse_worst = 0.0
    ar = torch.arange(64, device=dev)
    for b in range(B):
        qpos = (64 * int(past_blocks[b]) + torch.arange(Lq, device=dev)).repeat_interleave(G)  # rows t*G + g
        for hk in range(Hkv):
            r = b * Hkv + hk
            ids = tab[r, :int(cnt[r])].to(dev).long()
            keys = (ids[:, None] * 64 + ar[None, :]).reshape(-1)
            kf = k_hf[b, hk].index_select(0, keys).float()
            vf = v_hf[b, hk].index_select(0, keys).float()
            qf = q[b, :, hk * G:(hk + 1) * G].float().reshape(Lq * G, D)
            s = (qf @ kf.T.contiguous()) * scale
            s.masked_fill_(keys[None, :] > qpos[:, None], float("-inf"))
            ref_lse = torch.logsumexp(s, dim=-1)
            o = torch.softmax(s, dim=-1) @ vf
            del s
            got = out[b, :, hk * G:(hk + 1) * G].float().reshape(Lq * G, D)
            err = (got - o).abs()
            worst = max(worst, err.max().item())
            total += err.sum().item()
            n += err.numel()
            if lse is not None:
                got_lse = lse[b, hk * G:(hk + 1) * G].float().transpose(0, 1).reshape(-1)
                lse_worst = max(lse_worst, (got_lse - ref_lse).abs().max().item())
    mean = total / n
    assert worst <= atol_max and mean <= atol_mean, (worst, mean)
    assert lse_worst <= lse_atol, lse_worst
    return worst, mean


def ref_seer_tables(scores, past, Hkv, threshold, keep_recent_blocks, kv_group_aware=False):
    """Restatement of the reference's Seer selection for a chunk: _build_keep_block_mask_chunked_
    fast_path (compact_attn/modules/attention_forward_chunked_dense.py:559-638) -- past column kb
    kept iff the max over the query blocks of score[qb, kb] > threshold, current column j iff the
    max over the query blocks that see it (qb >= j, the suffix max at the diagonal) > threshold,
    then the last keep_recent_blocks of the Kb = P + Qb columns set -- and
    _build_kv_head_union_keep_block_mask (:641-683): the past columns OR-ed over the G heads of
    a KV group (a kv-group-aware gate's rows are the KV groups already), the current chunk open
    (and the preprojected path's current-open step, :1044-1050).  threshold is a float or a
    sequence with one value per request.  scores [B, Hs, Qb, >= P+Qb]; returns (table [B*Hkv,
    cap] -1 padded with cap = scores.shape[-1], counts)."""
    s_all = torch.as_tensor(np.asarray(scores), dtype=torch.float32)
    B, Hs, Qb, cap = s_all.shape
    G = 1 if kv_group_aware else Hs // Hkv
    thr = list(threshold) if isinstance(threshold, (list, tuple, np.ndarray)) else [float(threshold)] * B
    table = np.full((B * Hkv, cap), -1, np.int32)
    counts = np.zeros((B * Hkv,), np.int32)
    for b in range(B):
        P = int(past[b])
        Kb = P + Qb
        s = s_all[b, :, :, :Kb]
        keep_past = s[..., :P].amax(dim=1) > thr[b]
        curr = s[..., P:Kb]  # [H, Qb, Qb]
        suffix = torch.flip(torch.cummax(torch.flip(curr, dims=[1]), dim=1).values, dims=[1])
        j = torch.arange(Qb)
        keep_curr = suffix[:, j, j] > thr[b]
        keep = torch.cat([keep_past, keep_curr], dim=-1)
        recent = min(int(keep_recent_blocks), Kb)
        if recent > 0:
            keep[:, Kb - recent:] = True
        kv_past = keep[:, :P].view(Hkv, G, P).any(dim=1)
        kv = torch.cat([kv_past, torch.ones((Hkv, Qb), dtype=torch.bool)], dim=-1)
        for hk in range(Hkv):
            ids = torch.nonzero(kv[hk]).flatten().numpy()
            table[b * Hkv + hk, :len(ids)] = ids
            counts[b * Hkv + hk] = len(ids)
    return table, counts


def spy_union_compact(monkeypatch):
    """Records the (table, counts) of every ops.union_compact call the code under test makes."""
    from compactattention_amd import ops

    calls = []
    real = ops.union_compact

    def spy(*args, **kw):
        out = real(*args, **kw)
        calls.append((out[0].detach().clone(), out[1].detach().clone()))
        return out

    monkeypatch.setattr(ops, "union_compact", spy)
    return calls
