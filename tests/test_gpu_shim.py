"""The reference-side shim (compactattention_amd.native_shim) against torch restatements of the
reference's native kernels it stands in for (compact_attn/csrc/compactattn/cache_fill_kernel.cu):

  - build_keep_past_fast :275-298  -- per (b, h) and past column c: max over the query blocks
    of score[q][c] (NaN skipped, start -FLT_MAX) > threshold;
  - build_keep_curr_fast :301-326  -- per current column c: the same max over q >= c of
    score[q][P + c];
  - build_selected_indices_from_kv_keep_block :449-483 -- ascending kept ids and counts;
  - build_flashinfer_kv_indices :485-505 -- kv_indices[indptr[r] + i] = r * kv_blocks + ids[r][i].

Inputs carry ties at the threshold, NaN and -inf; every output is compared exactly.
"""
from __future__ import annotations

import pytest
import torch

from compactattention_amd import native_shim

pytestmark = pytest.mark.gpu


def _scores(B, H, Qb, P, dtype, seed, thr):
    g = torch.Generator().manual_seed(seed)
    s = torch.rand((B, H, Qb, P + Qb), generator=g) * (2 * thr)
    s[0, 0, 0, :3] = thr  # ties at the threshold are not kept (strict >)
    s[0, min(1, H - 1), Qb - 1, 1] = float("nan")
    s[-1, -1, 0, 2] = float("-inf")
    return s.to(dtype).cuda()


def _ref_keep_past(s, thr, P):
    x = s.float()[:, :, :, :P].nan_to_num(nan=float("-inf"))
    return x.amax(2) > thr


def _ref_keep_curr(s, thr, P, C):
    x = s.float()[:, :, :, P:P + C].nan_to_num(nan=float("-inf"))
    Qb = x.shape[2]
    q = torch.arange(Qb, device=x.device)[:, None]
    c = torch.arange(C, device=x.device)[None, :]
    x = x.masked_fill(q < c, float("-inf"))  # query block q sees current block c iff c <= q
    return x.amax(2) > thr


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,Qb,P", [(1, 4, 4, 37), (2, 8, 16, 300)])
def test_keep_past_and_curr_match_reference_kernels(gpu, dtype, B, H, Qb, P):
    print(f"case: shim keep masks dtype={dtype} B={B} H={H} Qb={Qb} P={P}", flush=True)
    thr = 0.01
    s = _scores(B, H, Qb, P, dtype, 7 + P, thr)
    past = native_shim.build_keep_past_fast_cuda(attn_gate_score=s, threshold=thr, past_k_blocks=P)
    curr = native_shim.build_keep_curr_fast_cuda(attn_gate_score=s, threshold=thr, past_k_blocks=P,
                                                 curr_k_blocks=Qb)
    torch.cuda.synchronize()
    assert past.dtype == torch.bool and past.shape == (B, H, P)
    assert torch.equal(past, _ref_keep_past(s, thr, P))
    assert curr.shape == (B, H, Qb)
    assert torch.equal(curr, _ref_keep_curr(s, thr, P, Qb))


@pytest.mark.parametrize("last_kept", [True, False])
def test_selected_indices_and_flashinfer_indices_match_reference_kernels(gpu, last_kept):
    print(f"case: shim selected indices last_kept={last_kept}", flush=True)
    B, Hkv, Kb = 2, 4, 133
    g = torch.Generator().manual_seed(11)
    keep = torch.rand((B, Hkv, Kb), generator=g) < 0.3
    keep[:, :, -1] = last_kept
    keep[1, 2] = False  # an empty row (or only the last block)
    keep = keep.cuda()
    cap = Kb + 5
    ids = torch.full((B * Hkv, cap), -7, dtype=torch.int32, device=gpu)
    counts = torch.empty((B * Hkv,), dtype=torch.int32, device=gpu)
    native_shim.build_selected_indices_from_kv_keep_block_cuda_out(keep_block_kv=keep, selected_block_indices=ids,
                                                                  selected_block_counts=counts)
    torch.cuda.synchronize()
    flat = keep.reshape(B * Hkv, Kb).cpu()
    for r in range(B * Hkv):
        want = torch.nonzero(flat[r]).flatten().to(torch.int32)
        assert int(counts[r]) == want.numel(), r
        assert torch.equal(ids[r, :want.numel()].cpu(), want), r

    # CSR page lists over the same rows, the caller building kv_indptr as the reference's do
    indptr = torch.zeros((B * Hkv + 1,), dtype=torch.int32, device=gpu)
    indptr[1:] = torch.cumsum(counts, 0)
    total = int(indptr[-1])
    kv_indices = torch.full((B * Hkv * Kb,), -3, dtype=torch.int32, device=gpu)
    native_shim.build_flashinfer_kv_indices_cuda_out(selected_block_indices=ids, selected_block_counts=counts,
                                                     kv_indptr=indptr, kv_indices=kv_indices, kv_blocks=Kb)
    torch.cuda.synchronize()
    want = torch.cat([r * Kb + torch.nonzero(flat[r]).flatten() for r in range(B * Hkv)]).to(torch.int32)
    assert torch.equal(kv_indices[:total].cpu(), want)


def test_gather_side_has_no_counterpart(gpu):
    assert native_shim.cuda_cache_fill_available()
    assert not native_shim.can_use_cuda_pack_q_for_indexed_prefill()
    assert not native_shim.can_use_cuda_compact_keep_blocks()
    with pytest.raises(NotImplementedError, match="in place"):
        native_shim.cache_fill_from_past_indices_cuda(k=None)
