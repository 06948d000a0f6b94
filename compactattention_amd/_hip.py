"""ctypes binding of libcompactattn_hip.so (the C-ABI declared in include/compactattn.h).

This module replaces the reference's extension loader
(compact_attn/kernels/varlen/indexed_dense_cache_fill_cuda.py:10-19), with one deliberate
difference: a missing or unloadable library raises instead of returning None, because
this build has no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcompactattn_hip.so")

ABI_VERSION = 2
HEAD_DIM = 128
BLOCK = 64
MAX_BATCH = 64
STATIC_SCRATCH_BYTES = 48 << 20

CA_OK = 0
CA_ERR_INVALID = -1
CA_ERR_LIMIT = -2
CA_ERR_WORKSPACE = -3
CA_ERR_HIP = -4

RULE_TOPK = 1
RULE_ALPHA = 2
RULE_THRESHOLD = 4
RULE_TOPK_ALLCOLS = 8

POOL_MAX = 1
POOL_MIN = 2
POOL_AVG = 4

EXPORTED = (
    "ca_abi_version",
    "ca_last_error",
    "ca_cache_fill",
    "ca_pool_query",
    "ca_cache_fill_pool_query",
    "ca_gate_key_summaries",
    "ca_gate_query_summaries",
    "ca_pair_block_summaries",
    "ca_score_select",
    "ca_score_token_mass",
    "ca_select_scores",
    "ca_union_compact",
    "ca_compact_keep_kv",
    "ca_dense_table",
    "ca_table_to_csr",
    "ca_attn_fwd",
    "ca_attn_workspace_size",
    "ca_attn_pick_splits",
    "ca_attn_fwd_noalloc",
    "ca_attn_decode",
    "ca_attn_decode_workspace_size",
    "ca_rope_apply",
    "ca_rmsnorm",
    "ca_swiglu",
)


class CaError(RuntimeError):
    """Raised when a C-ABI call returns a CA_ERR_* code."""

    def __init__(self, code: int, message: str):
        super().__init__(f"compactattn error {code}: {message}")
        self.code = code


class Dims(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("q_len", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("kv_cap", ctypes.c_int32),
    ]


class KvLayout(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_blk", ctypes.c_int64),
        ("stride_tok", ctypes.c_int64),
        ("page_table", ctypes.c_void_p),
        ("page_table_stride", ctypes.c_int64),
        ("num_pages", ctypes.c_int64),
    ]


class SeqLayout(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_t", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
    ]


class SelectRule(ctypes.Structure):
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


_P = ctypes.POINTER
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

_SIGNATURES = {
    "ca_abi_version": (ctypes.c_int, []),
    "ca_last_error": (ctypes.c_char_p, []),
    "ca_cache_fill": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _P(SeqLayout), _P(KvLayout), _P(KvLayout),
                                     _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "ca_pool_query": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "ca_cache_fill_pool_query": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _P(SeqLayout), _P(KvLayout), _P(KvLayout),
                                                _vp, _vp, _P(SeqLayout), _vp, _vp]),
    "ca_gate_key_summaries": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _vp, _i32, _vp, _i32, _vp, _vp, _i64, _vp,
                                             _vp]),
    "ca_gate_query_summaries": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _vp, _i32, _vp, _i32, _vp, _vp, _i64,
                                               _vp, _vp]),
    "ca_pair_block_summaries": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp]),
    "ca_score_select": (ctypes.c_int, [_P(Dims), _vp, _vp, _f32, _P(SelectRule), _vp, _vp, _vp, _vp]),
    "ca_score_token_mass": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _vp, _i64, _i32, _f32, _vp, _vp, _vp]),
    "ca_select_scores": (ctypes.c_int, [_P(Dims), _vp, _i32, _i64, _i64, _i64, _P(SelectRule), _vp, _vp, _vp]),
    "ca_union_compact": (ctypes.c_int, [_P(Dims), _vp, _i32, _vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "ca_compact_keep_kv": (ctypes.c_int, [_P(Dims), _vp, _vp, _vp, _i64, _vp, _vp]),
    "ca_dense_table": (ctypes.c_int, [_P(Dims), _vp, _vp, _i64, _vp, _vp]),
    "ca_table_to_csr": (ctypes.c_int, [_P(Dims), _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp]),
    "ca_attn_fwd": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _P(KvLayout), _P(KvLayout), _vp, _i64, _vp, _vp,
                                   _f32, _P(SeqLayout), _vp, _i32, _vp, _i64, _vp]),
    "ca_attn_workspace_size": (ctypes.c_int64, [_P(Dims), _vp, _i32]),
    "ca_attn_pick_splits": (ctypes.c_int32, [_P(Dims), _vp]),
    "ca_attn_fwd_noalloc": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _P(KvLayout), _P(KvLayout), _vp, _i64, _vp,
                                           _vp, _f32, _P(SeqLayout), _vp, _i32, _vp]),
    "ca_attn_decode": (ctypes.c_int, [_P(Dims), _P(SeqLayout), _P(KvLayout), _P(KvLayout), _vp, _f32,
                                      _P(SeqLayout), _vp, _i32, _vp, _i64, _vp]),
    "ca_attn_decode_workspace_size": (ctypes.c_int64, [_P(Dims), _vp, _i32]),
    "ca_rope_apply": (ctypes.c_int, [_P(SeqLayout), _P(SeqLayout), _i32, _i32, _i32, _vp, _vp, _vp]),
    "ca_rmsnorm": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i32, _f32, _vp]),
    "ca_swiglu": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _vp]),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it is missing (there is no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m compactattention_amd.build` "
                "(the compactattn path has no non-HIP fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        version = handle.ca_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}")
        _lib = handle
        return _lib


def last_error() -> str:
    msg = lib().ca_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc != CA_OK:
        raise CaError(rc, last_error())
