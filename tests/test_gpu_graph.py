"""GPU test: the whole chunk path (cache fill -> pooled scores -> selection -> Block-Union ->
indexed attention with split-KV merge) captured in one HIP graph and replayed gives the
eager path's results bit for bit on every replay, with eager work and synchronisations
between the replays.  The library records no memset or allocation, so the path is
capturable as called from Python (the benchmark times its stages this way)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from compactattention_amd import ops
from compactattention_amd.synthetic import make_chunk_device

from .util import bits

pytestmark = pytest.mark.gpu


def test_chunk_path_graph_replays_match_eager(gpu):
    print("case: chunk path graph capture, past 8192, chunk 256, 8 Q / 2 KV heads", flush=True)
    PAST, LQ, HQ, HKV = 8192, 256, 8, 2
    ch = make_chunk_device(PAST, LQ, HQ, HKV, gpu, seed=77)
    cap, P = ch.kv_cap, ch.past_blocks
    K, V = ops.KV.heads_first(ch.k), ops.KV.heads_first(ch.v)
    kmean = torch.zeros((1, HKV, cap, 128), dtype=torch.float32, device=gpu)
    scale = 1.0 / math.sqrt(128)
    # past summaries, then the chunk's K/V handed over seq-first
    for t0 in range(0, PAST, 4096):
        t1 = t0 + 4096
        ops.cache_fill(ch.k[:, :, t0:t1].transpose(1, 2).contiguous(), ch.v[:, :, t0:t1].transpose(1, 2).contiguous(),
                       K, V, [t0 // 64], cap, kmean)
    k_new = ch.k[:, :, PAST:PAST + LQ].transpose(1, 2).contiguous()
    v_new = ch.v[:, :, PAST:PAST + LQ].transpose(1, 2).contiguous()
    rule = ops.Rule(topk=6, sink_blocks=1, local_blocks=2)
    splits = 3
    ws = torch.empty((ops.attn_workspace_bytes(P, LQ, HQ, HKV, cap, splits),), dtype=torch.uint8, device=gpu)
    out = torch.empty_like(ch.q)

    def step():
        ops.cache_fill(k_new, v_new, K, V, P, cap, kmean)
        qhat = ops.pool_query(ch.q, P, cap)
        rowmask, _ = ops.score_select(qhat, kmean, scale, rule, P, HKV, cap)
        table, counts, _, _ = ops.union_compact(rowmask, P, HKV, cap)
        ops.attn_fwd(ch.q, K, V, table, counts, P, scale, cap, HKV, out=out, num_splits=splits, workspace=ws)
        return table, counts

    t_e, c_e = step()
    torch.cuda.synchronize()
    ref = {"out": bits(out), "table": t_e.cpu().numpy(), "counts": c_e.cpu().numpy(),
           "kmean": kmean.cpu().numpy(), "k": bits(ch.k)}

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        t_g, c_g = step()
    for rep in range(3):
        # eager work between replays: clobber the outputs the graph must rewrite
        out.fill_(0)
        kmean[:, :, P[0]:P[0] + LQ // 64].zero_()
        ch.k[:, :, PAST:PAST + LQ].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), ref["out"]), rep
        assert np.array_equal(t_g.cpu().numpy(), ref["table"]), rep
        assert np.array_equal(c_g.cpu().numpy(), ref["counts"]), rep
        assert np.array_equal(bits(ch.k), ref["k"]), rep
        kmean_now = kmean.cpu().numpy()
        live = ref["kmean"][:, :, :P[0] + LQ // 64]
        assert np.array_equal(kmean_now[:, :, :P[0] + LQ // 64].view(np.uint32), live.view(np.uint32)), rep
