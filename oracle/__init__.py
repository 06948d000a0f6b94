"""CPU oracle for the compactattn chunked-prefill path.

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use this package, and only as the
checker or the timed CPU baseline.  The product package ``compactattention_amd``
never imports it.

The numerics live in ``ca_oracle.c`` (fixed fp32 evaluation order, explicit
fmaf); this module is a numpy front end over ctypes.  bf16 tensors travel as
``np.uint16`` bit patterns.  One function is numpy fp64 instead:
``token_mass_scores`` (the reference's per-token FlashPrefill scores, which the product
computes on MFMAs and matches to a tolerance, not bit for bit).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libca_oracle.so")

RULE_TOPK = 1
RULE_ALPHA = 2
RULE_THRESHOLD = 4
RULE_TOPK_ALLCOLS = 8
D = 128
BLOCK = 64


class _Rule(ctypes.Structure):
    _fields_ = [
        ("flags", ctypes.c_int32),
        ("topk", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("threshold", ctypes.c_float),
        ("sink_blocks", ctypes.c_int32),
        ("window_blocks", ctypes.c_int32),
        ("local_blocks", ctypes.c_int32),
        ("last_n_block", ctypes.c_int32),
    ]


@dataclass
class Rule:
    """Selection rule; field meanings follow the product's ``ca_select_rule``."""

    topk: int = 0
    alpha: Optional[float] = None
    threshold: Optional[float] = None
    sink_blocks: int = 0
    window_blocks: int = 0
    local_blocks: int = 0
    last_n_block: int = 0
    topk_all_columns: bool = False  # rank all Kb columns (the reference's min_budget)

    def to_c(self) -> _Rule:
        flags = 0
        if self.topk > 0:
            flags |= RULE_TOPK
            if self.topk_all_columns:
                flags |= RULE_TOPK_ALLCOLS
        if self.alpha is not None:
            flags |= RULE_ALPHA
        if self.threshold is not None:
            flags |= RULE_THRESHOLD
        return _Rule(
            flags,
            int(self.topk),
            float(self.alpha if self.alpha is not None else 0.0),
            float(self.threshold if self.threshold is not None else 0.0),
            int(self.sink_blocks),
            int(self.window_blocks),
            int(self.local_blocks),
            int(self.last_n_block),
        )


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_exp.restype = ctypes.c_float
        _lib.orc_exp.argtypes = [ctypes.c_float]
        _lib.orc_num_threads.restype = ctypes.c_int
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(x: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(x, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def exp(x: np.ndarray) -> np.ndarray:
    f = lib().orc_exp
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in flat], dtype=np.float32).reshape(np.shape(x))


def block_mean(x_bits: np.ndarray) -> np.ndarray:
    """x: [B, L, H, 128] bf16 bits -> [B, H, ceil(L/64), 128] fp32 block means (a partial last
    block averages its L % 64 tokens)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    B, L, H, d = x.shape
    assert d == D and L > 0
    out = np.empty((B, H, -(-L // BLOCK), D), dtype=np.float32)
    lib().orc_block_mean(_p(x), B, L, H, _p(out))
    return out


POOL_MAX = 1
POOL_MIN = 2
POOL_AVG = 4
POOL_BITS = {"max": POOL_MAX, "min": POOL_MIN, "avg": POOL_AVG}


def pool_bits(names) -> int:
    """('max', 'avg') -> POOL_MAX | POOL_AVG (the concatenation order is always max, min, avg)."""
    bits_ = 0
    for nm in names:
        bits_ |= POOL_BITS[nm]
    return bits_


def block_pool(x_bits: np.ndarray, pools: int) -> np.ndarray:
    """x: [B, L, H, 128] bf16 bits -> [B, H, ceil(L/64), C*128] fp32 (max, min, avg as selected;
    a partial last block pools its L % 64 tokens)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    B, L, H, d = x.shape
    assert d == D and L > 0 and 0 < pools < 8
    C = bin(pools).count("1")
    out = np.empty((B, H, -(-L // BLOCK), C * D), dtype=np.float32)
    lib().orc_block_pool(_p(x), B, L, H, int(pools), _p(out))
    return out


def pair_block_means(src: np.ndarray, last_tokens: int) -> np.ndarray:
    """[..., n_blocks, 128] fp32 64-token summaries (the last block holding last_tokens tokens)
    -> [..., ceil(n_blocks/2), 128] 128-token summaries."""
    x = np.ascontiguousarray(src, dtype=np.float32)
    lead, n = x.shape[:-2], x.shape[-2]
    rows = int(np.prod(lead)) if lead else 1
    out = np.empty(lead + (-(-n // 2), D), dtype=np.float32)
    lib().orc_pair_block_means(_p(x), rows, n, int(last_tokens), _p(out))
    return out


def gate_project(x: np.ndarray, W: np.ndarray, cos: Optional[np.ndarray], sin: Optional[np.ndarray],
                 first_block) -> np.ndarray:
    """x: [B, H, N, in] fp32; W: [H, in, 128]; cos/sin: [rows, 128] by absolute block id."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    B, H, N, width = x.shape
    assert W.shape == (H, width, D)
    fb = _i32(first_block)
    y = np.empty((B, H, N, D), dtype=np.float32)
    if cos is None:
        lib().orc_gate_project_n(_p(x), B, H, N, width, _p(W), None, None, ctypes.c_int64(0), _p(fb), _p(y))
    else:
        c = np.ascontiguousarray(cos, dtype=np.float32)
        s = np.ascontiguousarray(sin, dtype=np.float32)
        lib().orc_gate_project_n(_p(x), B, H, N, width, _p(W), _p(c), _p(s), ctypes.c_int64(c.shape[0]),
                                 _p(fb), _p(y))
    return y


def block_scores(qhat: np.ndarray, khat: np.ndarray, past_blocks, scale: float) -> np.ndarray:
    """qhat [B,Hq,Qb,128], khat [B,Hkv,cap,128] -> softmax-normalised scores [B,Hq,Qb,cap]."""
    qhat = np.ascontiguousarray(qhat, dtype=np.float32)
    khat = np.ascontiguousarray(khat, dtype=np.float32)
    B, Hq, Qb, _ = qhat.shape
    _, Hkv, cap, _ = khat.shape
    pb = _i32(past_blocks)
    out = np.empty((B, Hq, Qb, cap), dtype=np.float32)
    lib().orc_block_scores(_p(qhat), _p(khat), B, Hq, Hkv, Qb, cap, _p(pb), ctypes.c_float(scale), _p(out))
    return out


def token_mass_scores(q_bits: np.ndarray, khat: np.ndarray, past_blocks, scale: float, block_size: int,
                      kv_cap: int) -> np.ndarray:
    """FlashPrefill per-token block scores in fp64, restating compute_block_score_chunked with
    K_STRIDE = BLOCK_SIZE (compact_attn/flashprefill_vendor/flashprefill_native_forward.py:98-207)
    and normalize_scores (:365-374).

    q_bits [B, Lq, Hq, 128] bf16 bits; khat [B, Hkv, >= nk, 128] fp32 block means, rounded to
    bf16 as the reference stores mean_k (:436-443); past_blocks in block_size-token blocks.  For
    query block qb the token slots t < block_size sit at absolute positions
    start + qb*BS + t (start = P*BS; slots past Lq hold zero queries, :159-163); key block kb is
    scored for kb < hi = min(ceil((qmax + 1) / BS), nk) (:166) and seen by slot t when
    start + qb*BS + t >= kb*BS + BS - 1 (:175-177).  Returns [B, Hq, ceil(Lq/BS), kv_cap]
    float64 (0 past nk)."""
    q = bf16_bits_to_f32(q_bits).astype(np.float64)
    kb16 = bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(khat, dtype=np.float32))).astype(np.float64)
    B, Lq, Hq, _ = q.shape
    Hkv = kb16.shape[1]
    G = Hq // Hkv
    BS = int(block_size)
    Qb = -(-Lq // BS)
    sm = float(scale) * 1.4426950408889634
    out = np.zeros((B, Hq, Qb, kv_cap), dtype=np.float64)
    for b in range(B):
        P = int(past_blocks[b])
        start = P * BS
        nk = P + Qb
        for h in range(Hq):
            kbf = kb16[b, h // G]
            for qb in range(Qb):
                qt = np.zeros((BS, D))
                n_valid = min(BS, Lq - qb * BS)
                qt[:n_valid] = q[b, qb * BS:qb * BS + n_valid, h]
                qabs = start + qb * BS + np.arange(BS)
                qmax = start + qb * BS + BS - 1
                hi = min(-(-(qmax + 1) // BS), nk)
                m = np.full(kv_cap, -np.inf)
                mass = np.zeros(kv_cap)
                if hi > 0:
                    s = (qt @ kbf[:hi].T) * sm  # [BS, hi]
                    causal = qabs[:, None] >= (np.arange(hi) * BS + BS - 1)[None, :]
                    s = np.where(causal, s, -np.inf)
                    mk = s.max(axis=0)
                    with np.errstate(invalid="ignore"):
                        e = np.where(causal, np.exp2(s - mk[None, :]), 0.0)
                    m[:hi] = mk
                    mass[:hi] = e.sum(axis=0)
                ok = m[:nk] != -np.inf
                M = m[:nk].max()
                sc = np.where(ok, mass[:nk] * np.exp2(np.where(ok, m[:nk] - M, 0.0)), 0.0)
                out[b, h, qb, :nk] = sc / (sc.sum() + 1e-9)
    return out


def select_rows(scores: np.ndarray, past_blocks, rule: Rule) -> np.ndarray:
    s = np.ascontiguousarray(scores, dtype=np.float32)
    B, Hq, Qb, cap = s.shape
    pb = _i32(past_blocks)
    out = np.empty((B, Hq, Qb, cap), dtype=np.uint8)
    r = rule.to_c()
    lib().orc_select_rows(_p(s), B, Hq, Qb, cap, _p(pb), ctypes.byref(r), _p(out))
    return out


def union_compact(rowkeep: np.ndarray, Hkv: int, past_blocks, last_n_block: int = 0
                  ) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """-> keep_block [B,Hq,cap] u8, keep_kv [B,Hkv,cap] u8, table [B*Hkv,cap] i32, counts [B*Hkv]."""
    rk = np.ascontiguousarray(rowkeep, dtype=np.uint8)
    B, Hq, Qb, cap = rk.shape
    pb = _i32(past_blocks)
    keep_block = np.empty((B, Hq, cap), dtype=np.uint8)
    keep_kv = np.empty((B, Hkv, cap), dtype=np.uint8)
    table = np.empty((B * Hkv, cap), dtype=np.int32)
    counts = np.empty((B * Hkv,), dtype=np.int32)
    lib().orc_union_compact(_p(rk), B, Hq, Hkv, Qb, cap, _p(pb), int(last_n_block), _p(keep_block),
                            _p(keep_kv), _p(table), _p(counts))
    return keep_block, keep_kv, table, counts


def attention(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, past_blocks, table: np.ndarray,
              counts: np.ndarray, scale: float, q_range: Optional[Tuple[int, int]] = None,
              head_range: Optional[Tuple[int, int]] = None, with_lse: bool = False):
    """q [B,Lq,Hq,128] bf16 bits; k,v [B,Hkv,cap*64,128] bf16 bits heads-first.

    Returns out [B,Lq,Hq,128] fp32 (and lse [B,Hq,Lq] if requested).  Entries outside
    q_range / head_range are NaN.
    """
    q = np.ascontiguousarray(q_bits, dtype=np.uint16)
    k = np.ascontiguousarray(k_bits, dtype=np.uint16)
    v = np.ascontiguousarray(v_bits, dtype=np.uint16)
    B, Lq, Hq, _ = q.shape
    _, Hkv, ktok, _ = k.shape
    cap = ktok // BLOCK
    tab = np.ascontiguousarray(table, dtype=np.int32)
    assert tab.shape[1] == cap, "table stride must equal the KV capacity in blocks"
    cnt = _i32(counts)
    pb = _i32(past_blocks)
    q0, q1 = q_range if q_range is not None else (0, Lq)
    h0, h1 = head_range if head_range is not None else (0, Hq)
    out = np.full((B, Lq, Hq, D), np.nan, dtype=np.float32)
    lse = np.full((B, Hq, Lq), np.nan, dtype=np.float32) if with_lse else None
    lib().orc_attention(_p(q), _p(k), _p(v), B, Lq, Hq, Hkv, cap, _p(pb), _p(tab), _p(cnt),
                        ctypes.c_float(scale), q0, q1, h0, h1, _p(out),
                        _p(lse) if lse is not None else None)
    return (out, lse) if with_lse else out


def attention_decode(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, kv_len, scale: float,
                     with_lse: bool = False):
    """Dense causal attention of each request's q_len newest tokens over its whole cache.

    The reference routes decode (q_len == 1) to dense attention over the updated cache
    (compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:878-894 ->
    compact_attn/modules/dense_prefill.py:117-175, flash_attn_func with causal=True).  With
    q_len < kv_len that causal mask is aligned bottom-right: query row t sits at position
    kv_len - q_len + t and sees keys 0 .. kv_len - q_len + t.  Inputs are bf16 bit patterns,
    the arithmetic is fp64 (numpy); tokens at or past kv_len[b] are never read.

    q [B, Lq, Hq, 128]; k, v [B, Hkv, >= max(kv_len), 128] heads-first.  Returns out
    [B, Lq, Hq, 128] fp32 (and lse [B, Hq, Lq], natural log, if requested).
    """
    B, Lq, Hq, _ = q_bits.shape
    Hkv = k_bits.shape[1]
    G = Hq // Hkv
    q = bf16_bits_to_f32(q_bits).astype(np.float64)
    out = np.zeros((B, Lq, Hq, D), dtype=np.float32)
    lse = np.zeros((B, Hq, Lq), dtype=np.float32)
    t = np.arange(Lq)
    for b in range(B):
        n = int(kv_len[b])
        pos = n - Lq + t  # absolute position of query row t
        visible = np.arange(n)[None, :] <= pos[:, None]  # [Lq, n]
        for hk in range(Hkv):
            k = bf16_bits_to_f32(k_bits[b, hk, :n]).astype(np.float64)
            v = bf16_bits_to_f32(v_bits[b, hk, :n]).astype(np.float64)
            for g in range(G):
                hq = hk * G + g
                s = (q[b, :, hq] @ k.T) * scale
                s = np.where(visible, s, -np.inf)
                m = s.max(axis=1, keepdims=True)
                p = np.exp(s - m)
                l = p.sum(axis=1, keepdims=True)
                out[b, :, hq] = (p @ v) / l
                lse[b, hq] = (m + np.log(l))[:, 0]
    return (out, lse) if with_lse else out


def num_threads() -> int:
    return int(lib().orc_num_threads())
