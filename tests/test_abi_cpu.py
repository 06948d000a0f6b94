"""The C-ABI library on the CPU: it loads, exports every entry point the header declares,
and its host-side validation rejects bad arguments before any launch (no GPU needed).
Also the Python entry points' argument errors."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from compactattention_amd import _hip, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "compactattn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ca_[a-z_0-9]+)\s*\(", text)))


def test_header_matches_exports():
    names = declared_functions()
    assert set(names) == set(_hip.EXPORTED), names
    out = subprocess.run(["nm", "-D", "--defined-only", _hip.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (ca_[a-z_0-9]+)\b", out))
    assert set(names) <= exported, set(names) - exported


def test_library_loads_and_reports_version():
    lib = _hip.lib()
    assert lib.ca_abi_version() == _hip.ABI_VERSION == 2


def _dims(**kw):
    d = dict(batch=1, q_len=128, num_q_heads=8, num_kv_heads=2, kv_cap=10)
    d.update(kw)
    return _hip.Dims(d["batch"], d["q_len"], d["num_q_heads"], d["num_kv_heads"], d["kv_cap"])


FAKE = 1 << 20  # a 16-byte aligned address never dereferenced (validation fails first)


def _seq(data=FAKE, sb=0, st=1024, sh=128):
    return _hip.SeqLayout(data, sb, st, sh)


def _kv(data=FAKE, sb=0, sh=0, sblk=8192, stok=128):
    return _hip.KvLayout(data, sb, sh, sblk, stok, None, 0, 0)


def _past(*p):
    return (ctypes.c_int32 * len(p))(*p)


@pytest.mark.parametrize("dims,past,code,msg", [
    (_dims(batch=0), (0,), _hip.CA_ERR_INVALID, "batch"),
    (_dims(batch=65), (0,), _hip.CA_ERR_LIMIT, "batch"),
    (_dims(q_len=0), (0,), _hip.CA_ERR_INVALID, "must be positive"),
    (_dims(q_len=100, kv_cap=1), (0,), _hip.CA_ERR_INVALID, "exceeds kv_cap"),  # 100 tokens span 2 blocks
    (_dims(num_q_heads=7), (0,), _hip.CA_ERR_INVALID, "multiple"),
    (_dims(num_q_heads=34, num_kv_heads=2), (0,), _hip.CA_ERR_LIMIT, "group size"),
    (_dims(kv_cap=9), (8,), _hip.CA_ERR_INVALID, "exceeds kv_cap"),
    (_dims(), (-1,), _hip.CA_ERR_INVALID, "< 0"),
])
def test_dims_validation(dims, past, code, msg):
    lib = _hip.lib()
    rc = lib.ca_attn_fwd(ctypes.byref(dims), ctypes.byref(_seq()), ctypes.byref(_kv()), ctypes.byref(_kv()), FAKE,
                         16, FAKE, _past(*past), 0.1, ctypes.byref(_seq()), None, 1, None, 0, None)
    assert rc == code
    assert msg in _hip.last_error()


def test_layout_and_workspace_validation():
    lib = _hip.lib()
    d = _dims()
    args = lambda q, k, split, ws, wsb, scale=0.1, tstride=16: lib.ca_attn_fwd(  # noqa: E731
        ctypes.byref(d), ctypes.byref(q), ctypes.byref(k), ctypes.byref(_kv()), FAKE, tstride, FAKE, _past(0),
        scale, ctypes.byref(_seq()), None, split, ws, wsb, None)
    assert args(_seq(data=FAKE + 2), _kv(), 1, None, 0) == _hip.CA_ERR_INVALID
    assert "aligned" in _hip.last_error()
    assert args(_seq(st=1023), _kv(), 1, None, 0) == _hip.CA_ERR_INVALID
    assert args(_seq(), _kv(stok=0), 1, None, 0) == _hip.CA_ERR_INVALID
    assert args(_seq(), _kv(), 1, None, 0, tstride=4) == _hip.CA_ERR_INVALID
    assert args(_seq(), _kv(), 1, None, 0, scale=0.0) == _hip.CA_ERR_INVALID
    assert args(_seq(), _kv(), 17, None, 0) == _hip.CA_ERR_INVALID
    assert args(_seq(), _kv(), 2, None, 0) == _hip.CA_ERR_WORKSPACE
    need = lib.ca_attn_workspace_size(ctypes.byref(d), _past(0), 2)
    # splits * B*Hkv * Lq*G rows * 129 floats, then a 16-byte flag slot
    assert need == 2 * 1 * 2 * 128 * 4 * 129 * 4 + 16
    assert args(_seq(), _kv(), 2, FAKE, need - 1) == _hip.CA_ERR_WORKSPACE
    assert lib.ca_attn_pick_splits(ctypes.byref(d), _past(0)) >= 1


@pytest.mark.parametrize("B,lq,hq,hkv,past,expect", [
    (1, 1024, 32, 8, 2048, 2),  # config 2: 128 row tiles, one round of 256 work items
    (1, 256, 32, 8, 128, 8),    # config 0: 32 row tiles (also the 16-blocks-per-split floor)
    (1, 2048, 32, 8, 1024, 1),  # a config-3 chunk: 256 row tiles fill the CUs unsplit
    (1, 512, 28, 4, 256, 4),    # 56 row tiles: 4 splits (224 items), not 5 (280: two rounds)
    (1, 1024, 24, 6, 2048, 2),  # 96 row tiles: 2 splits (192 items), not 3 (288)
])
def test_prefill_automatic_split_count(B, lq, hq, hkv, past, expect):
    """Requests of one length get the largest split count whose work items fit one round of
    the 256 CUs (none when the row tiles alone fill three quarters of them)."""
    d = _dims(batch=B, q_len=lq, num_q_heads=hq, num_kv_heads=hkv, kv_cap=past + lq // 64)
    n = _hip.lib().ca_attn_pick_splits(ctypes.byref(d), _past(*([past] * B)))
    assert n == expect
    units = B * hkv * -(-lq * (hq // hkv) // 256)
    assert n == 1 or n * units <= 256


@pytest.mark.parametrize("kv,expect", [
    ([1024], 4),       # 16 blocks: the floor of 4 blocks per split
    ([4096], 16),      # 64 blocks: 4 per split, 128 work items
    ([16384], 32),     # 256 blocks: the cap of 32 splits, 256 work items
    ([131072], 32),    # 2048 blocks: 64 per split, 256 work items
    ([4096] * 4, 8),   # 32 KV rows x 8 splits = 256 work items
    ([64], 1),         # one block: no split, no workspace
])
def test_decode_automatic_split_count(kv, expect):
    """Decode's per-request plan (32 Q / 8 KV heads, one token): about 256 work items, at least
    4 blocks per split, at most 32 splits; read back from the workspace size it asks for."""
    B, hq, hkv = len(kv), 32, 8
    d = _dims(batch=B, q_len=1, num_q_heads=hq, num_kv_heads=hkv, kv_cap=(max(kv) + 63) // 64)
    need = _hip.lib().ca_attn_decode_workspace_size(ctypes.byref(d), _past(*kv), 0)
    rows = B * hkv * (hq // hkv)
    splits = 1 if need == 0 else (need - 16) // (rows * 129 * 4)
    assert need == 0 or need == splits * rows * 129 * 4 + 16
    assert splits == expect


@pytest.mark.parametrize("dims,kv_len,code,msg", [
    (_dims(batch=0), (1,), _hip.CA_ERR_INVALID, "batch"),
    (_dims(q_len=0), (1,), _hip.CA_ERR_INVALID, "q_len"),
    (_dims(q_len=65), (100,), _hip.CA_ERR_INVALID, "q_len"),
    (_dims(q_len=1, num_q_heads=34, num_kv_heads=2), (8,), _hip.CA_ERR_LIMIT, "group size"),
    (_dims(q_len=4), (3,), _hip.CA_ERR_INVALID, "kv_len[0]"),
    (_dims(q_len=1, kv_cap=2), (129,), _hip.CA_ERR_INVALID, "kv_len[0]"),
    (_dims(q_len=1, kv_cap=0), (1,), _hip.CA_ERR_INVALID, "kv_cap"),
])
def test_decode_dims_validation(dims, kv_len, code, msg):
    lib = _hip.lib()
    rc = lib.ca_attn_decode(ctypes.byref(dims), ctypes.byref(_seq()), ctypes.byref(_kv()), ctypes.byref(_kv()),
                            _past(*kv_len), 0.1, ctypes.byref(_seq()), None, 1, None, 0, None)
    assert rc == code
    assert msg in _hip.last_error()


def test_decode_layout_and_workspace_validation():
    lib = _hip.lib()
    d = _dims(batch=2, q_len=1, kv_cap=100)
    kv = _past(70, 6400)
    call = lambda q, split, ws, wsb, scale=0.1, kvl=kv: lib.ca_attn_decode(  # noqa: E731
        ctypes.byref(d), ctypes.byref(q), ctypes.byref(_kv()), ctypes.byref(_kv()), kvl, scale,
        ctypes.byref(_seq()), None, split, ws, wsb, None)
    assert call(_seq(data=FAKE + 2), 1, None, 0) == _hip.CA_ERR_INVALID
    assert call(_seq(), 1, None, 0, scale=-1.0) == _hip.CA_ERR_INVALID
    assert call(_seq(), 65, None, 0) == _hip.CA_ERR_INVALID
    assert call(_seq(), 4, None, 0) == _hip.CA_ERR_WORKSPACE
    assert call(_seq(), 0, None, 0) == _hip.CA_ERR_WORKSPACE  # a 100-block row is split by the plan
    need = lib.ca_attn_decode_workspace_size(ctypes.byref(d), kv, 4)
    assert need == 4 * 2 * 2 * (1 * 4) * 129 * 4 + 16  # splits * B*Hkv * Lq*G rows * 129 floats + flag
    assert call(_seq(), 4, FAKE, need - 1) == _hip.CA_ERR_WORKSPACE
    assert lib.ca_attn_decode_workspace_size(ctypes.byref(d), kv, 0) > 0
    assert lib.ca_attn_decode_workspace_size(ctypes.byref(d), kv, 65) < 0
    # one request of one block needs no split and no workspace
    d1 = _dims(batch=1, q_len=1, kv_cap=1)
    assert lib.ca_attn_decode_workspace_size(ctypes.byref(d1), _past(64), 0) == 0


def test_table_to_csr_validation():
    lib = _hip.lib()
    d = _dims(batch=2, num_kv_heads=2, kv_cap=10)
    call = lambda stride, cap_idx, dd=d: lib.ca_table_to_csr(ctypes.byref(dd), FAKE, stride, FAKE, FAKE, FAKE,  # noqa: E731
                                                            cap_idx, None, None)
    assert call(9, 40) == _hip.CA_ERR_INVALID and "table_stride" in _hip.last_error()
    assert call(10, 39) == _hip.CA_ERR_INVALID and "indices_capacity" in _hip.last_error()
    big = _dims(batch=64, num_kv_heads=129, kv_cap=10)
    assert call(10, 1 << 30, big) == _hip.CA_ERR_LIMIT
    rc = lib.ca_table_to_csr(ctypes.byref(d), None, 10, FAKE, FAKE, FAKE, 40, None, None)
    assert rc == _hip.CA_ERR_INVALID


def test_rule_and_select_validation():
    lib = _hip.lib()
    d = _dims()
    bad = _hip.SelectRule(16, 0, 0.0, 0.0, 0, 0, 0, 0)
    rc = lib.ca_select_scores(ctypes.byref(d), FAKE, 0, 0, 0, 0, ctypes.byref(bad), _past(2), FAKE, None)
    assert rc == _hip.CA_ERR_INVALID and "flags" in _hip.last_error()
    # the all-columns modifier needs the top-k rule itself
    lone = _hip.SelectRule(_hip.RULE_TOPK_ALLCOLS, 3, 0.0, 0.0, 0, 0, 0, 0)
    rc = lib.ca_select_scores(ctypes.byref(d), FAKE, 0, 0, 0, 0, ctypes.byref(lone), _past(2), FAKE, None)
    assert rc == _hip.CA_ERR_INVALID and "CA_RULE_TOPK" in _hip.last_error()
    neg = _hip.SelectRule(_hip.RULE_TOPK, -1, 0.0, 0.0, 0, 0, 0, 0)
    rc = lib.ca_select_scores(ctypes.byref(d), FAKE, 0, 0, 0, 0, ctypes.byref(neg), _past(2), FAKE, None)
    assert rc == _hip.CA_ERR_INVALID
    ok = _hip.SelectRule(0, 0, 0.0, 0.0, 0, 0, 0, 0)
    rc = lib.ca_select_scores(ctypes.byref(d), FAKE, 2, 0, 0, 0, ctypes.byref(ok), _past(2), FAKE, None)
    assert rc == _hip.CA_ERR_INVALID and "dtype" in _hip.last_error()
    rc = lib.ca_score_select(ctypes.byref(d), FAKE, FAKE, 0.1, ctypes.byref(ok), _past(2), FAKE, None, None)
    assert rc == _hip.CA_ERR_INVALID and "scores" in _hip.last_error()
    rc = lib.ca_union_compact(ctypes.byref(d), FAKE, 0, _past(2), None, None, FAKE, 4, FAKE, None)
    assert rc == _hip.CA_ERR_INVALID and "table_stride" in _hip.last_error()


def test_cache_fill_validation():
    lib = _hip.lib()
    d = _dims()
    rc = lib.ca_cache_fill(ctypes.byref(d), ctypes.byref(_seq()), None, None, None, _past(0), None, None, None, None,
                           0, None, None)
    assert rc == _hip.CA_ERR_INVALID and "nothing to do" in _hip.last_error()
    rc = lib.ca_cache_fill(ctypes.byref(d), ctypes.byref(_seq()), ctypes.byref(_seq()), ctypes.byref(_kv()),
                           ctypes.byref(_kv()), _past(0), FAKE, FAKE, None, None, 0, None, None)
    assert rc == _hip.CA_ERR_INVALID and "kgate" in _hip.last_error()
    pt = _hip.KvLayout(FAKE, 0, 0, 8192, 128, FAKE, 1, 8)
    rc = lib.ca_cache_fill(ctypes.byref(d), ctypes.byref(_seq()), ctypes.byref(_seq()), ctypes.byref(pt),
                           ctypes.byref(_kv()), _past(0), FAKE, None, None, None, 0, None, None)
    assert rc == _hip.CA_ERR_INVALID and "page_table_stride" in _hip.last_error()
    # a page table needs the pool's page count (ids are clamped into it)
    nopages = _hip.KvLayout(FAKE, 0, 0, 8192, 128, FAKE, 10, 0)
    rc = lib.ca_cache_fill(ctypes.byref(d), ctypes.byref(_seq()), ctypes.byref(_seq()), ctypes.byref(nopages),
                           ctypes.byref(_kv()), _past(0), FAKE, None, None, None, 0, None, None)
    assert rc == _hip.CA_ERR_INVALID and "num_pages" in _hip.last_error()


def test_token_stride_limit():
    """The kernels address a block's 64 rows with 32-bit byte offsets: stride_tok >= 2^24 is
    refused (CA_ERR_LIMIT) by every entry point that reads or writes a KV layout."""
    lib = _hip.lib()
    d = _dims()
    big = _kv(stok=1 << 24, sblk=64 << 24)
    rc = lib.ca_cache_fill(ctypes.byref(d), ctypes.byref(_seq()), ctypes.byref(_seq()), ctypes.byref(big),
                           ctypes.byref(_kv()), _past(0), FAKE, None, None, None, 0, None, None)
    assert rc == _hip.CA_ERR_LIMIT and "stride_tok" in _hip.last_error()
    ok = _kv(stok=(1 << 24) - 8, sblk=64 * ((1 << 24) - 8))
    rc = lib.ca_attn_fwd(ctypes.byref(d), ctypes.byref(_seq()), ctypes.byref(big), ctypes.byref(ok), FAKE, 10, FAKE,
                         _past(0), 0.1, ctypes.byref(_seq()), None, 1, None, 0, None)
    assert rc == _hip.CA_ERR_LIMIT and "stride_tok" in _hip.last_error()
    kvl = (ctypes.c_int32 * 1)(100)
    rc = lib.ca_attn_decode(ctypes.byref(_dims(q_len=1)), ctypes.byref(_seq()), ctypes.byref(ok), ctypes.byref(big),
                            kvl, 0.1, ctypes.byref(_seq()), None, 1, None, 0, None)
    assert rc == _hip.CA_ERR_LIMIT and "stride_tok" in _hip.last_error()


def test_gate_summary_validation():
    lib = _hip.lib()
    d = _dims()  # Hq 8, Hkv 2
    call_k = lambda pools, heads, w=FAKE, out=FAKE: lib.ca_gate_key_summaries(  # noqa: E731
        ctypes.byref(d), ctypes.byref(_seq()), _past(0), pools, w, heads, None, None, 0, out, None)
    assert call_k(0, 2) == _hip.CA_ERR_INVALID and "pools" in _hip.last_error()
    assert call_k(8, 2) == _hip.CA_ERR_INVALID and "pools" in _hip.last_error()
    assert call_k(7, 3) == _hip.CA_ERR_INVALID and "gate_heads" in _hip.last_error()
    assert call_k(7, 2, w=None) == _hip.CA_ERR_INVALID
    call_q = lambda pools, heads, w=FAKE: lib.ca_gate_query_summaries(  # noqa: E731
        ctypes.byref(d), ctypes.byref(_seq()), _past(0), pools, w, heads, None, None, 0, FAKE, None)
    # several pools need a projection; an unprojected summary has one head per Q head
    assert call_q(_hip.POOL_MAX | _hip.POOL_AVG, 8, w=None) == _hip.CA_ERR_INVALID and "projection" in _hip.last_error()
    assert call_q(_hip.POOL_AVG, 2, w=None) == _hip.CA_ERR_INVALID and "gate_heads" in _hip.last_error()
    assert call_q(_hip.POOL_AVG, 4) == _hip.CA_ERR_INVALID and "gate_heads" in _hip.last_error()


def test_python_entry_points_reject_bad_arguments():
    from compactattention_amd.modules.attention_forward_chunked_dense import (
        chunked_prefill_column_dense_attention_forward, chunked_prefill_column_dense_attention_from_keep_block)
    from compactattention_amd.modules.flashprefill_prefill import flashprefill_compactattn_prefill_full_kv

    q = torch.zeros((1, 128, 8, 128), dtype=torch.bfloat16)
    k = torch.zeros((1, 640, 2, 128), dtype=torch.bfloat16)
    gate = torch.zeros((1, 8, 2, 10))
    f = chunked_prefill_column_dense_attention_forward
    with pytest.raises(ValueError, match="attn_gate_score is required"):
        f(q, k, k, None, 128)
    with pytest.raises(ValueError, match="query_length > 1"):
        f(q, k, k, None, 1, attn_gate_score=gate)
    with pytest.raises(ValueError, match="block_size must be positive"):
        f(q, k, k, None, 128, attn_gate_score=gate, block_size=0)
    with pytest.raises(ValueError, match="Unsupported indexed_impl"):
        f(q, k, k, None, 128, attn_gate_score=gate, indexed_impl="nope")
    with pytest.raises(ValueError, match="64-token blocks"):
        f(q, k, k, None, 128, attn_gate_score=gate, block_size=128, num_key_value_groups=4)
    # an unaligned call splits into an aligned head and a dense tail; its chunk must start on a block
    with pytest.raises(ValueError, match="block boundary"):
        f(q, k[:, :600], k[:, :600], None, 128, attn_gate_score=gate, num_key_value_groups=4)
    with pytest.raises(ValueError, match="does not match query_states"):
        f(q[:, :100], k, k, None, 128, attn_gate_score=gate, num_key_value_groups=4)
    with pytest.raises(ValueError, match="threshold tensor has 2 values for a batch of 1"):
        f(q, k, k, None, 128, attn_gate_score=gate, threshold=torch.zeros(2), num_key_value_groups=4)
    with pytest.raises(ValueError, match="Expected scalar or 1D batch threshold tensor"):
        f(q, k, k, None, 128, attn_gate_score=gate, threshold=torch.zeros((1, 1)), num_key_value_groups=4)
    with pytest.raises(ValueError, match="Either keep_block"):
        chunked_prefill_column_dense_attention_from_keep_block(q, k, k, None, None, 128, 0.1,
                                                               num_key_value_groups=4)
    with pytest.raises(ValueError, match="keep_block shape mismatch"):
        chunked_prefill_column_dense_attention_from_keep_block(q, k, k, torch.zeros((1, 8, 9), dtype=torch.bool),
                                                               None, 128, 0.1, num_key_value_groups=4)
    with pytest.raises(ValueError, match="Unsupported indexed_impl"):
        flashprefill_compactattn_prefill_full_kv(
            q, k, k, None, softmax_scale=0.1, num_key_value_groups=4, block_size=64, attention_sink=2,
            window_size=4, alpha=0.06, last_n_block=0, min_budget=0, pack_impl="torch", indexed_impl="x",
            cache_fill_backend="auto")
    with pytest.raises(ValueError, match="padded positions"):
        mask = torch.ones((1, 640), dtype=torch.bool)
        mask[0, 3] = False
        f(q, k, k, mask, 128, attn_gate_score=gate, num_key_value_groups=4)


def test_ops_reject_cpu_tensors():
    q = torch.zeros((1, 128, 8, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.pool_query(q, [0], 2)


def test_model_plumbing_validation():
    lib = _hip.lib()
    x = _seq(FAKE, 64 * 8 * 128, 8 * 128, 128)
    assert lib.ca_rope_apply(ctypes.byref(x), ctypes.byref(x), 0, 64, 8, FAKE, FAKE, None) == _hip.CA_ERR_INVALID
    assert lib.ca_rope_apply(ctypes.byref(x), ctypes.byref(x), 1, 64, 8, None, FAKE, None) == _hip.CA_ERR_INVALID
    assert "cos" in _hip.last_error()
    rms = lambda n, rows=4, res=0, s=0, eps=1e-5: lib.ca_rmsnorm(FAKE, n, res, n, s, n, FAKE, FAKE, n,  # noqa: E731
                                                                 rows, n, eps, None)
    assert rms(12) == _hip.CA_ERR_INVALID and "n=12" in _hip.last_error()
    assert rms(64, res=FAKE) == _hip.CA_ERR_INVALID and "together" in _hip.last_error()
    assert rms(64, eps=-1.0) == _hip.CA_ERR_INVALID
    assert rms(64, rows=1 << 31) == _hip.CA_ERR_LIMIT
    assert rms(64, rows=0, res=FAKE, s=FAKE) == _hip.CA_OK  # nothing to launch
    assert lib.ca_rmsnorm(FAKE, 64, 0, 0, 0, 0, FAKE + 2, FAKE, 64, 4, 64, 1e-5, None) == _hip.CA_ERR_INVALID
    swi = lambda n, gs, rows=4: lib.ca_swiglu(FAKE, gs, FAKE, n, FAKE, n, rows, n, None)  # noqa: E731
    assert swi(4, 4) == _hip.CA_ERR_INVALID
    assert swi(64, 32) == _hip.CA_ERR_INVALID and "strides" in _hip.last_error()
    assert swi(64, 128, rows=0) == _hip.CA_OK
    assert lib.ca_swiglu(None, 64, FAKE, 64, FAKE, 64, 4, 64, None) == _hip.CA_ERR_INVALID


def test_model_plumbing_python_errors():
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises((ValueError, RuntimeError)):
        ops.rmsnorm(x, torch.ones(64, dtype=torch.bfloat16), 1e-5)
    with pytest.raises((ValueError, RuntimeError)):
        ops.swiglu(x, x)
    with pytest.raises((ValueError, RuntimeError)):
        ops.rope(torch.zeros((1, 64, 2, 128), dtype=torch.bfloat16), torch.zeros(64, 128), torch.zeros(64, 128))
