"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the oracle
reproduces them on the CPU, and the HIP kernels reproduce them on the GPU (bit-exact
summaries, scores, selections and tables; attention within the north-star tolerance)."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle

from .util import f32, float_bits_equal, unpack_rowmask

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


def test_oracle_reproduces_golden():
    m = load("golden_mean.npz")
    assert float_bits_equal(oracle.block_mean(m["k_bits"]), m["means"])
    g = load("golden_gate.npz")
    assert float_bits_equal(oracle.gate_project(g["x"], g["W"], g["cos"], g["sin"], g["first_block"]), g["y"])
    s = load("golden_select.npz")
    sc = oracle.block_scores(s["qhat"], s["khat"], s["past"], float(s["scale"]))
    assert float_bits_equal(sc, s["scores"])
    kt = oracle.select_rows(sc, s["past"], oracle.Rule(topk=3, sink_blocks=1, local_blocks=2))
    assert np.array_equal(kt, s["keep_topk"])
    assert np.array_equal(oracle.select_rows(sc, s["past"], oracle.Rule(alpha=0.5, sink_blocks=2, window_blocks=4)),
                          s["keep_alpha"])
    _, kv, table, counts = oracle.union_compact(kt, 2, s["past"])
    assert np.array_equal(kv, s["keep_kv"]) and np.array_equal(table, s["table"])
    assert np.array_equal(counts, s["counts"])
    a = load("golden_attention.npz")
    out, lse = oracle.attention(a["q_bits"], a["k_bits"], a["v_bits"], a["past"], a["table"], a["counts"],
                                float(a["scale"]), with_lse=True)
    assert np.abs(out - a["out"]).max() <= 1e-6 and np.abs(lse - a["lse"]).max() <= 1e-6


@pytest.mark.gpu
def test_kernels_reproduce_golden(gpu):
    from compactattention_amd import ops

    print("case: golden fixtures", flush=True)
    m = load("golden_mean.npz")
    k = torch.from_numpy(m["k_bits"].view(np.int16)).view(torch.bfloat16).to(gpu)
    kmean = torch.zeros((1, 1, 2, 128), dtype=torch.float32, device=gpu)
    ops.cache_fill(k, None, None, None, [0], 2, kmean)
    assert float_bits_equal(f32(kmean), m["means"])

    s = load("golden_select.npz")
    past = [int(p) for p in s["past"]]
    qhat = torch.from_numpy(s["qhat"]).to(gpu)
    khat = torch.from_numpy(s["khat"].reshape(2, 12, 128)).to(gpu)
    rule = ops.Rule(topk=3, sink_blocks=1, local_blocks=2)
    rowmask, scores = ops.score_select(qhat, khat, float(s["scale"]), rule, past, 2, 12, with_scores=True)
    assert float_bits_equal(f32(scores), s["scores"])
    assert np.array_equal(unpack_rowmask(rowmask, 12), s["keep_topk"])
    table, counts, _, keep_kv = ops.union_compact(rowmask, past, 2, 12, want_keep_kv=True)
    assert np.array_equal(table.cpu().numpy(), s["table"]) and np.array_equal(counts.cpu().numpy(), s["counts"])
    assert np.array_equal(keep_kv.cpu().numpy(), s["keep_kv"])

    a = load("golden_attention.npz")
    to = lambda x: torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(gpu)  # noqa: E731
    out, lse = ops.attn_fwd(to(a["q_bits"]), ops.KV.heads_first(to(a["k_bits"])), ops.KV.heads_first(to(a["v_bits"])),
                            torch.from_numpy(a["table"]).to(gpu), torch.from_numpy(a["counts"]).to(gpu),
                            [int(p) for p in a["past"]], float(a["scale"]), 3, 1, with_lse=True)
    err = np.abs(f32(out) - a["out"])
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
