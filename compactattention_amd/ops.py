"""Torch-tensor front end of the C-ABI (one function per entry point).

Each wrapper checks devices/dtypes, builds the layout structs from tensor strides and
launches on ``torch.cuda.current_stream()``.  Outputs are allocated with torch's caching
allocator here (the C-ABI itself never allocates).  Nothing in this module falls back to
a non-HIP implementation.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from . import _hip
from ._hip import BLOCK, HEAD_DIM, POOL_AVG, POOL_MAX, POOL_MIN, Dims, KvLayout, SelectRule, SeqLayout, check

POOL_BITS = {"max": POOL_MAX, "min": POOL_MIN, "avg": POOL_AVG}


def pool_bits(names: Sequence[str]) -> int:
    """Pool names ('max', 'min', 'avg') -> CA_POOL_* bits; the kernels concatenate the pooled
    vectors in the order max, min, avg, the order of the reference's generated gate classes
    (itertools.combinations over ['max', 'min', 'avg'], attn_gate.py:265-278)."""
    out = 0
    for nm in names:
        if nm not in POOL_BITS:
            raise ValueError(f"unknown pooling function {nm!r}")
        out |= POOL_BITS[nm]
    order = [nm for nm in ("max", "min", "avg") if nm in names]
    if list(names) != order or not names:
        raise ValueError(f"pooling functions {tuple(names)} must be a non-empty subset of ('max', 'min', 'avg') "
                         "in that order")
    return out


@dataclass(frozen=True)
class Rule:
    """Block selection rule (``ca_select_rule``).

    topk       keep the top-k past blocks of every (head, query block) row, ordered by
               (score desc, block id asc);
    topk_all_columns
               rank every column kb < P + Qb instead (non-causal and non-finite entries
               read as 0) and keep the causal picks -- the reference's ``min_budget``
               (torch.topk over the zeroed row, flashprefill_prefill.py:633-647);
    alpha      keep blocks with score >= alpha * row max (FlashPrefill);
    threshold  keep blocks with score > threshold (SeerAttention, strict);
    sink_blocks / window_blocks / local_blocks / last_n_block as in ``ca_select_rule``.
    """

    topk: int = 0
    alpha: Optional[float] = None
    threshold: Optional[float] = None
    sink_blocks: int = 0
    window_blocks: int = 0
    local_blocks: int = 0
    last_n_block: int = 0
    topk_all_columns: bool = False

    def to_c(self) -> SelectRule:
        flags = 0
        if self.topk > 0:
            flags |= _hip.RULE_TOPK
            if self.topk_all_columns:
                flags |= _hip.RULE_TOPK_ALLCOLS
        if self.alpha is not None:
            flags |= _hip.RULE_ALPHA
        if self.threshold is not None:
            flags |= _hip.RULE_THRESHOLD
        return SelectRule(
            flags,
            int(self.topk),
            float(self.alpha if self.alpha is not None else 0.0),
            float(self.threshold if self.threshold is not None else 0.0),
            int(self.sink_blocks),
            int(self.window_blocks),
            int(self.local_blocks),
            int(self.last_n_block),
        )


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need_cuda(name: str, t: torch.Tensor, dtype: torch.dtype) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")


def past_array(past_blocks: Sequence[int], batch: Optional[int] = None):
    """Per-request values (past blocks or kv_len) as the int32 host array the C-ABI reads
    ``batch`` entries of."""
    vals = [int(x) for x in past_blocks]
    if not 1 <= len(vals) <= _hip.MAX_BATCH:
        raise ValueError(f"batch must be in [1, {_hip.MAX_BATCH}]")
    if batch is not None and len(vals) != batch:
        raise ValueError(f"{len(vals)} per-request values for a batch of {batch}")
    return (ctypes.c_int32 * len(vals))(*vals)


def make_dims(batch: int, q_len: int, num_q_heads: int, num_kv_heads: int, kv_cap: int) -> Dims:
    return Dims(int(batch), int(q_len), int(num_q_heads), int(num_kv_heads), int(kv_cap))


def seq_layout(t: torch.Tensor, name: str = "tensor") -> SeqLayout:
    """[B, T, H, 128] bf16 with a contiguous head dim."""
    _need_cuda(name, t, torch.bfloat16)
    if t.dim() != 4 or t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
        raise ValueError(f"{name} must be [B, T, H, {HEAD_DIM}] with a contiguous last dim")
    return SeqLayout(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


@dataclass
class KV:
    """A K or V tensor plus the way 64-token blocks are addressed in it."""

    tensor: torch.Tensor
    layout: KvLayout
    page_table: Optional[torch.Tensor] = None
    tokens: Optional[int] = None  # token capacity of a contiguous layout (None when paged)
    batch: Optional[int] = None   # requests of a contiguous layout (None when paged)
    heads: Optional[int] = None   # KV heads of a contiguous layout (None when paged)

    @staticmethod
    def seq_first(t: torch.Tensor) -> "KV":
        """[B, K, Hkv, 128] (the reference's key_states/value_states)."""
        _need_cuda("kv", t, torch.bfloat16)
        if t.dim() != 4 or t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
            raise ValueError("seq-first KV must be [B, K, Hkv, 128] with a contiguous last dim")
        return KV(t, KvLayout(t.data_ptr(), t.stride(0), t.stride(2), BLOCK * t.stride(1), t.stride(1), None, 0,
                              0), tokens=t.shape[1], batch=t.shape[0], heads=t.shape[2])

    @staticmethod
    def heads_first(t: torch.Tensor) -> "KV":
        """[B, Hkv, K, 128] (the reference's k_hf/v_hf cache)."""
        _need_cuda("kv", t, torch.bfloat16)
        if t.dim() != 4 or t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
            raise ValueError("heads-first KV must be [B, Hkv, K, 128] with a contiguous last dim")
        return KV(t, KvLayout(t.data_ptr(), t.stride(0), t.stride(1), BLOCK * t.stride(2), t.stride(2), None, 0,
                              0), tokens=t.shape[2], batch=t.shape[0], heads=t.shape[1])

    @staticmethod
    def paged(pool: torch.Tensor, page_table: torch.Tensor) -> "KV":
        """Global page pool [num_pages, 64, 128] and page_table [B*Hkv, blocks] int32."""
        _need_cuda("pool", pool, torch.bfloat16)
        _need_cuda("page_table", page_table, torch.int32)
        if pool.dim() != 3 or pool.shape[1] != BLOCK or pool.shape[2] != HEAD_DIM or pool.stride(-1) != 1:
            raise ValueError("page pool must be [num_pages, 64, 128]")
        if page_table.dim() != 2 or page_table.stride(1) != 1:
            raise ValueError("page_table must be [rows, blocks] with contiguous rows")
        return KV(pool, KvLayout(pool.data_ptr(), 0, 0, pool.stride(0), pool.stride(1), page_table.data_ptr(),
                                 page_table.stride(0), pool.shape[0]), page_table)

    def check_blocks(self, name: str, batch: int, heads: int, blocks: int, tokens: Optional[int] = None) -> None:
        """Raise unless this layout covers ``blocks`` logical blocks of each of the ``batch`` x
        ``heads`` KV rows: page-table rows and columns, or for a contiguous cache its requests,
        heads and whole 64-token blocks (``tokens`` tokens instead when the kernel's reads stop
        at that length)."""
        need = BLOCK * blocks if tokens is None else tokens
        if self.batch is not None and (self.batch < batch or self.heads < heads):
            raise ValueError(f"{name} cache holds {self.batch} requests x {self.heads} KV heads; the call "
                             f"addresses {batch} x {heads}")
        if self.tokens is not None and self.tokens < need:
            raise ValueError(f"{name} cache holds {self.tokens} tokens; the call addresses {blocks} blocks "
                             f"({need} tokens)")
        if self.page_table is not None:
            rows = batch * heads
            if self.page_table.shape[0] < rows or self.page_table.shape[1] < blocks:
                raise ValueError(f"{name} page_table {tuple(self.page_table.shape)} does not cover "
                                 f"[{rows}, {blocks}]")


def cache_fill(k_new: torch.Tensor, v_new: Optional[torch.Tensor], k_cache: Optional[KV], v_cache: Optional[KV],
               past_blocks: Sequence[int], kv_cap: int, kmean: Optional[torch.Tensor],
               gate_wk: Optional[torch.Tensor] = None, rope_cos: Optional[torch.Tensor] = None,
               rope_sin: Optional[torch.Tensor] = None, kgate: Optional[torch.Tensor] = None) -> None:
    """Append [B, Lq, Hkv, 128] K/V into the cache at past_blocks; write mean-K (and gate-K).

    With k_cache and v_cache None only the summaries are computed (nothing is copied)."""
    B, Lq, Hkv, _ = k_new.shape
    d = make_dims(B, Lq, Hkv, Hkv, kv_cap)
    kn = seq_layout(k_new, "k_new")
    if (k_cache is None) != (v_cache is None):
        raise ValueError("k_cache and v_cache must both be given or both be None")
    vn = seq_layout(v_new, "v_new") if k_cache is not None else None
    if vn is not None and tuple(v_new.shape) != tuple(k_new.shape):
        raise ValueError("v_new must have k_new's shape")
    blocks = max(int(p) for p in past_blocks) + -(-Lq // BLOCK)  # highest block written + 1
    tokens = BLOCK * max(int(p) for p in past_blocks) + Lq  # a partial last block writes its Lq % 64 rows
    for name, kv in (("k", k_cache), ("v", v_cache)):
        if kv is not None:
            kv.check_blocks(name, B, Hkv, blocks, tokens=tokens)
    if kmean is not None:
        _need_cuda("kmean", kmean, torch.float32)
        if not kmean.is_contiguous() or kmean.numel() < B * Hkv * kv_cap * HEAD_DIM:
            raise ValueError("kmean must be contiguous [B*Hkv, kv_cap, 128] fp32")
    rope_rows = 0
    if gate_wk is not None:
        _need_cuda("gate_wk", gate_wk, torch.float32)
        if tuple(gate_wk.shape) != (Hkv, HEAD_DIM, HEAD_DIM) or not gate_wk.is_contiguous():
            raise ValueError("gate_wk must be contiguous [Hkv, 128, 128] fp32")
        if kgate is None:
            raise ValueError("kgate output is required with gate_wk")
        _need_cuda("kgate", kgate, torch.float32)
        if not kgate.is_contiguous() or kgate.numel() < B * Hkv * kv_cap * HEAD_DIM:
            raise ValueError("kgate must be contiguous [B*Hkv, kv_cap, 128] fp32")
        if rope_cos is not None:
            _need_cuda("rope_cos", rope_cos, torch.float32)
            _need_cuda("rope_sin", rope_sin, torch.float32)
            rope_rows = rope_cos.shape[0]
    check(_hip.lib().ca_cache_fill(ctypes.byref(d), ctypes.byref(kn), ctypes.byref(vn) if vn is not None else None,
                                   ctypes.byref(k_cache.layout) if k_cache is not None else None,
                                   ctypes.byref(v_cache.layout) if v_cache is not None else None,
                                   past_array(past_blocks, d.batch), _ptr(kmean), _ptr(gate_wk), _ptr(rope_cos),
                                   _ptr(rope_sin), rope_rows, _ptr(kgate), _stream()))


def pool_query(q: torch.Tensor, past_blocks: Sequence[int], kv_cap: int, gate_wq: Optional[torch.Tensor] = None,
               rope_cos: Optional[torch.Tensor] = None, rope_sin: Optional[torch.Tensor] = None,
               num_kv_heads: Optional[int] = None) -> torch.Tensor:
    """[B, Lq, Hq, 128] bf16 -> qhat [B, Hq, ceil(Lq/64), 128] fp32."""
    B, Lq, Hq, _ = q.shape
    d = make_dims(B, Lq, Hq, num_kv_heads or Hq, kv_cap)
    ql = seq_layout(q, "q")
    rope_rows = 0
    if gate_wq is not None:
        _need_cuda("gate_wq", gate_wq, torch.float32)
        if tuple(gate_wq.shape) != (Hq, HEAD_DIM, HEAD_DIM) or not gate_wq.is_contiguous():
            raise ValueError("gate_wq must be contiguous [Hq, 128, 128] fp32")
        if rope_cos is not None:
            _need_cuda("rope_cos", rope_cos, torch.float32)
            _need_cuda("rope_sin", rope_sin, torch.float32)
            rope_rows = rope_cos.shape[0]
    qhat = torch.empty((B, Hq, -(-Lq // BLOCK), HEAD_DIM), dtype=torch.float32, device=q.device)
    check(_hip.lib().ca_pool_query(ctypes.byref(d), ctypes.byref(ql), past_array(past_blocks, d.batch), _ptr(gate_wq),
                                   _ptr(rope_cos), _ptr(rope_sin), rope_rows, qhat.data_ptr(), _stream()))
    return qhat


def cache_fill_pool_query(k_new: torch.Tensor, v_new: torch.Tensor, k_cache: KV, v_cache: KV,
                          past_blocks: Sequence[int], kv_cap: int, kmean: torch.Tensor,
                          q: torch.Tensor) -> torch.Tensor:
    """cache_fill(k_new, v_new, k_cache, v_cache, past_blocks, kv_cap, kmean) and
    pool_query(q, past_blocks, kv_cap) in one launch; returns qhat [B, Hq, ceil(Lq/64), 128] fp32."""
    B, Lq, Hkv, _ = k_new.shape
    Hq = q.shape[2]
    if tuple(q.shape[:2]) != (B, Lq) or tuple(v_new.shape) != tuple(k_new.shape):
        raise ValueError("q, k_new and v_new must cover the same [B, Lq] tokens")
    if Hq % Hkv:
        raise ValueError(f"num_q_heads={Hq} must be a multiple of num_kv_heads={Hkv}")
    d = make_dims(B, Lq, Hq, Hkv, kv_cap)
    kn, vn, ql = seq_layout(k_new, "k_new"), seq_layout(v_new, "v_new"), seq_layout(q, "q")
    blocks = max(int(p) for p in past_blocks) + -(-Lq // BLOCK)
    tokens = BLOCK * max(int(p) for p in past_blocks) + Lq
    k_cache.check_blocks("k", B, Hkv, blocks, tokens=tokens)
    v_cache.check_blocks("v", B, Hkv, blocks, tokens=tokens)
    _need_cuda("kmean", kmean, torch.float32)
    if not kmean.is_contiguous() or kmean.numel() < B * Hkv * kv_cap * HEAD_DIM:
        raise ValueError("kmean must be contiguous [B*Hkv, kv_cap, 128] fp32")
    qhat = torch.empty((B, Hq, -(-Lq // BLOCK), HEAD_DIM), dtype=torch.float32, device=q.device)
    check(_hip.lib().ca_cache_fill_pool_query(ctypes.byref(d), ctypes.byref(kn), ctypes.byref(vn),
                                              ctypes.byref(k_cache.layout), ctypes.byref(v_cache.layout),
                                              past_array(past_blocks, d.batch), kmean.data_ptr(), ctypes.byref(ql),
                                              qhat.data_ptr(), _stream()))
    return qhat


def _rope_args(rope_cos: Optional[torch.Tensor], rope_sin: Optional[torch.Tensor]) -> int:
    if (rope_cos is None) != (rope_sin is None):
        raise ValueError("rope_cos and rope_sin must both be given or both be None")
    if rope_cos is None:
        return 0
    for name, t in (("rope_cos", rope_cos), ("rope_sin", rope_sin)):
        _need_cuda(name, t, torch.float32)
        if t.dim() != 2 or t.shape[1] != HEAD_DIM or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous fp32 [rows, {HEAD_DIM}]")
    return rope_cos.shape[0]


def pool_count(pools: int) -> int:
    return bin(int(pools) & 7).count("1")


def gate_key_summaries(k_new: torch.Tensor, past_blocks: Sequence[int], kv_cap: int, pools: int,
                       gate_wk: torch.Tensor, kgate: torch.Tensor, num_q_heads: Optional[int] = None,
                       rope_cos: Optional[torch.Tensor] = None, rope_sin: Optional[torch.Tensor] = None) -> None:
    """AttnGate K summaries of the chunk's blocks: pools (POOL_* bits, concatenated max, min,
    avg) -> per-head projection gate_wk [gate_heads, C*128, 128] -> block RoPE, written into
    kgate [B, gate_heads, kv_cap, 128] at blocks past_blocks[b]...  gate_heads is Hkv or the
    number of Q heads (the K block repeated to each Q head of its group)."""
    B, Lq, Hkv, _ = k_new.shape
    Hq = num_q_heads or Hkv
    kn = seq_layout(k_new, "k_new")
    _need_cuda("gate_wk", gate_wk, torch.float32)
    _need_cuda("kgate", kgate, torch.float32)
    gh = gate_wk.shape[0]
    if gate_wk.dim() != 3 or tuple(gate_wk.shape[1:]) != (pool_count(pools) * HEAD_DIM, HEAD_DIM) \
            or not gate_wk.is_contiguous():
        raise ValueError(f"gate_wk must be contiguous [heads, {pool_count(pools) * HEAD_DIM}, {HEAD_DIM}] fp32")
    if not kgate.is_contiguous() or kgate.numel() < B * gh * kv_cap * HEAD_DIM:
        raise ValueError(f"kgate must be contiguous [B, {gh}, kv_cap, 128] fp32")
    rows = _rope_args(rope_cos, rope_sin)
    d = make_dims(B, Lq, Hq, Hkv, kv_cap)
    check(_hip.lib().ca_gate_key_summaries(ctypes.byref(d), ctypes.byref(kn), past_array(past_blocks, d.batch),
                                           int(pools), gate_wk.data_ptr(), gh, _ptr(rope_cos), _ptr(rope_sin), rows,
                                           kgate.data_ptr(), _stream()))


def gate_query_summaries(q: torch.Tensor, past_blocks: Sequence[int], kv_cap: int, pools: int,
                         gate_wq: Optional[torch.Tensor], num_kv_heads: int,
                         rope_cos: Optional[torch.Tensor] = None,
                         rope_sin: Optional[torch.Tensor] = None) -> torch.Tensor:
    """AttnGate query summaries: [B, Lq, Hq, 128] bf16 -> [B, gate_heads, ceil(Lq/64), 128] fp32.
    gate_wq None: one pool, no projection (gate_heads = Hq).  gate_wq [Hq, C*128, 128]: per
    Q head.  gate_wq [Hkv, G*C*128, 128]: the kv-group-aware form (the group's G heads
    pooled and concatenated head-major, one output per KV head)."""
    B, Lq, Hq, _ = q.shape
    ql = seq_layout(q, "q")
    C = pool_count(pools)
    G = Hq // num_kv_heads
    if gate_wq is None:
        gh = Hq
    else:
        _need_cuda("gate_wq", gate_wq, torch.float32)
        gh = gate_wq.shape[0]
        width = (G if (gh == num_kv_heads and G > 1) else 1) * C * HEAD_DIM
        if gate_wq.dim() != 3 or tuple(gate_wq.shape[1:]) != (width, HEAD_DIM) or not gate_wq.is_contiguous():
            raise ValueError(f"gate_wq must be contiguous [{gh}, {width}, {HEAD_DIM}] fp32")
    rows = _rope_args(rope_cos, rope_sin)
    d = make_dims(B, Lq, Hq, num_kv_heads, kv_cap)
    qhat = torch.empty((B, gh, -(-Lq // BLOCK), HEAD_DIM), dtype=torch.float32, device=q.device)
    check(_hip.lib().ca_gate_query_summaries(ctypes.byref(d), ctypes.byref(ql), past_array(past_blocks, d.batch),
                                             int(pools), _ptr(gate_wq), gh, _ptr(rope_cos), _ptr(rope_sin), rows,
                                             qhat.data_ptr(), _stream()))
    return qhat


def pair_block_summaries(src: torch.Tensor, n_blocks: int, last_tokens: int,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """64-token summaries [..., >= n_blocks, 128] fp32 (the last of the n_blocks holding
    last_tokens tokens) -> 128-token summaries [..., ceil(n_blocks/2), 128]:
    (c0 m0 + c1 m1) / (c0 + c1) per pair, an unpaired last block copied."""
    _need_cuda("src", src, torch.float32)
    if src.dim() < 2 or src.shape[-1] != HEAD_DIM or src.shape[-2] < n_blocks or src.stride(-1) != 1 \
            or src.stride(-2) != HEAD_DIM:
        raise ValueError("src must be [..., >= n_blocks, 128] with contiguous summaries")
    lead = src.shape[:-2]
    rows = 1
    for n in lead:
        rows *= int(n)
    src_rows = src.reshape(rows, src.shape[-2], HEAD_DIM)  # a view for the layouts the callers pass
    npairs = -(-int(n_blocks) // 2)
    if out is None:
        out = torch.empty((*lead, npairs, HEAD_DIM), dtype=torch.float32, device=src.device)
    dst_rows = out.reshape(rows, out.shape[-2], HEAD_DIM)
    if dst_rows.data_ptr() != out.data_ptr() or out.shape[-2] < npairs:
        raise ValueError("out must be contiguous [..., >= ceil(n_blocks/2), 128]")
    check(_hip.lib().ca_pair_block_summaries(src_rows.data_ptr(), src_rows.stride(0) // HEAD_DIM,
                                             dst_rows.data_ptr(), dst_rows.stride(0) // HEAD_DIM, rows,
                                             int(n_blocks), int(last_tokens), _stream()))
    return out


def words_for(kv_cap: int) -> int:
    return (kv_cap + 31) // 32


def score_select(qhat: torch.Tensor, khat: torch.Tensor, scale: float, rule: Rule, past_blocks: Sequence[int],
                 num_kv_heads: int, kv_cap: int, with_scores: bool = False
                 ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """qhat [B,Hq,Qb,128], khat [B*Hkv, kv_cap, 128] -> rowmask [B,Hq,Qb,words] (+ scores)."""
    _need_cuda("qhat", qhat, torch.float32)
    _need_cuda("khat", khat, torch.float32)
    if not qhat.is_contiguous() or not khat.is_contiguous():
        raise ValueError("qhat and khat must be contiguous")
    if qhat.dim() != 4 or qhat.shape[3] != HEAD_DIM:
        raise ValueError(f"qhat must be [B, Hq, Qb, {HEAD_DIM}]")
    B, Hq, Qb, _ = qhat.shape
    if khat.numel() < B * num_kv_heads * kv_cap * HEAD_DIM:
        raise ValueError("khat smaller than [B*Hkv, kv_cap, 128]")
    d = make_dims(B, Qb * BLOCK, Hq, num_kv_heads, kv_cap)
    rowmask = torch.empty((B, Hq, Qb, words_for(kv_cap)), dtype=torch.int32, device=qhat.device)
    scores = torch.empty((B, Hq, Qb, kv_cap), dtype=torch.float32, device=qhat.device)
    r = rule.to_c()
    check(_hip.lib().ca_score_select(ctypes.byref(d), qhat.data_ptr(), khat.data_ptr(), float(scale), ctypes.byref(r),
                                     past_array(past_blocks, d.batch), rowmask.data_ptr(), scores.data_ptr(),
                                     _stream()))
    return rowmask, (scores if with_scores else None)


def score_token_mass(q: torch.Tensor, khat: torch.Tensor, scale: float, past_blocks: Sequence[int], num_kv_heads: int,
                     kv_cap: int, block_size: int = 64) -> torch.Tensor:
    """FlashPrefill per-token block scores (ca_score_token_mass): q [B, Lq, Hq, 128] bf16 and key
    means khat [B*Hkv or B x Hkv, >= kv_cap, 128] fp32 in block_size-token blocks; past_blocks
    and kv_cap count block_size blocks.  Returns [B, Hq, ceil(Lq/block_size), kv_cap] fp32."""
    _need_cuda("khat", khat, torch.float32)
    if khat.shape[-1] != HEAD_DIM or khat.stride(-1) != 1 or khat.stride(-2) != HEAD_DIM:
        raise ValueError("khat must hold contiguous rows of 128-float block means")
    B, Lq, Hq, _ = q.shape
    rows = B * num_kv_heads
    stride_blocks = khat.stride(-3) // HEAD_DIM if khat.dim() >= 3 else kv_cap
    if khat.numel() < rows * stride_blocks * HEAD_DIM or not khat.is_contiguous():
        raise ValueError("khat must be contiguous [B*Hkv, blocks, 128]")
    d = make_dims(B, Lq, Hq, num_kv_heads, kv_cap)
    ql = seq_layout(q, "q")
    qb = -(-Lq // block_size)
    scores = torch.empty((B, Hq, qb, kv_cap), dtype=torch.float32, device=q.device)
    check(_hip.lib().ca_score_token_mass(ctypes.byref(d), ctypes.byref(ql), khat.data_ptr(), int(stride_blocks),
                                         int(block_size), float(scale), past_array(past_blocks, d.batch),
                                         scores.data_ptr(), _stream()))
    return scores


def select_scores(scores: torch.Tensor, rule: Rule, past_blocks: Sequence[int], num_kv_heads: int, kv_cap: int,
                  q_len: int) -> torch.Tensor:
    """Caller scores [B, Hq, Qb, >= P+Qb] (fp32 or bf16, last dim contiguous) -> rowmask."""
    if not scores.is_cuda:
        raise ValueError("scores must be a GPU tensor")
    if scores.dtype == torch.float32:
        dtype = 0
    elif scores.dtype == torch.bfloat16:
        dtype = 1
    else:
        raise ValueError(f"scores must be fp32 or bf16 (got {scores.dtype})")
    if scores.dim() != 4 or scores.stride(-1) != 1:
        raise ValueError("scores must be [B, Hq, Qb, Kb] with a contiguous last dim")
    B, Hq, Qb, Kb = scores.shape
    if Qb != -(-q_len // BLOCK):
        raise ValueError(f"scores have {Qb} query blocks, expected {-(-q_len // BLOCK)}")
    if Kb < max(int(p) for p in past_blocks) + Qb:
        raise ValueError("scores have fewer key blocks than past + current blocks")
    d = make_dims(B, q_len, Hq, num_kv_heads, kv_cap)
    rowmask = torch.empty((B, Hq, Qb, words_for(kv_cap)), dtype=torch.int32, device=scores.device)
    r = rule.to_c()
    check(_hip.lib().ca_select_scores(ctypes.byref(d), scores.data_ptr(), dtype, scores.stride(0), scores.stride(1),
                                      scores.stride(2), ctypes.byref(r), past_array(past_blocks, d.batch),
                                      rowmask.data_ptr(), _stream()))
    return rowmask


def union_compact(rowmask: torch.Tensor, past_blocks: Sequence[int], num_kv_heads: int, kv_cap: int,
                  last_n_block: int = 0, want_keep_block: bool = False, want_keep_kv: bool = False):
    """rowmask [B,Hq,Qb,words] -> (table [B*Hkv, kv_cap] i32, counts [B*Hkv] i32, keep_block, keep_kv)."""
    _need_cuda("rowmask", rowmask, torch.int32)
    if rowmask.dim() != 4 or rowmask.shape[3] != words_for(kv_cap) or not rowmask.is_contiguous():
        raise ValueError(f"rowmask must be contiguous [B, Hq, Qb, {words_for(kv_cap)}] int32")
    B, Hq, Qb, _ = rowmask.shape
    d = make_dims(B, Qb * BLOCK, Hq, num_kv_heads, kv_cap)
    dev = rowmask.device
    table = torch.empty((B * num_kv_heads, kv_cap), dtype=torch.int32, device=dev)
    counts = torch.empty((B * num_kv_heads,), dtype=torch.int32, device=dev)
    keep_block = torch.empty((B, Hq, kv_cap), dtype=torch.uint8, device=dev) if want_keep_block else None
    keep_kv = torch.empty((B, num_kv_heads, kv_cap), dtype=torch.uint8, device=dev) if want_keep_kv else None
    check(_hip.lib().ca_union_compact(ctypes.byref(d), rowmask.data_ptr(), int(last_n_block),
                                      past_array(past_blocks, d.batch), _ptr(keep_block), _ptr(keep_kv),
                                      table.data_ptr(), table.stride(0), counts.data_ptr(), _stream()))
    return table, counts, keep_block, keep_kv


def compact_keep_kv(keep_kv: torch.Tensor, past_blocks: Sequence[int], q_len: int, num_q_heads: int,
                    kv_cap: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """keep_kv [B, Hkv, kv_cap] u8/bool -> (table, counts); current-chunk blocks always kept."""
    if keep_kv.dtype == torch.bool:
        keep_kv = keep_kv.view(torch.uint8)
    _need_cuda("keep_kv", keep_kv, torch.uint8)
    B, Hkv, cap = keep_kv.shape
    if cap != kv_cap or not keep_kv.is_contiguous():
        raise ValueError("keep_kv must be contiguous [B, Hkv, kv_cap]")
    d = make_dims(B, q_len, num_q_heads, Hkv, kv_cap)
    table = torch.empty((B * Hkv, kv_cap), dtype=torch.int32, device=keep_kv.device)
    counts = torch.empty((B * Hkv,), dtype=torch.int32, device=keep_kv.device)
    check(_hip.lib().ca_compact_keep_kv(ctypes.byref(d), keep_kv.data_ptr(), past_array(past_blocks, d.batch),
                                        table.data_ptr(), table.stride(0), counts.data_ptr(), _stream()))
    return table, counts


def dense_table(past_blocks: Sequence[int], q_len: int, num_q_heads: int, num_kv_heads: int, kv_cap: int,
                device) -> Tuple[torch.Tensor, torch.Tensor]:
    B = len(past_blocks)
    d = make_dims(B, q_len, num_q_heads, num_kv_heads, kv_cap)
    table = torch.empty((B * num_kv_heads, kv_cap), dtype=torch.int32, device=device)
    counts = torch.empty((B * num_kv_heads,), dtype=torch.int32, device=device)
    check(_hip.lib().ca_dense_table(ctypes.byref(d), past_array(past_blocks, d.batch), table.data_ptr(),
                                    table.stride(0), counts.data_ptr(), _stream()))
    return table, counts


def table_to_csr(table: torch.Tensor, counts: torch.Tensor, batch: int, num_kv_heads: int, kv_cap: int,
                 with_last_page_len: bool = False):
    """Block tables -> (kv_indptr [rows+1], kv_indices [rows*kv_cap] (first kv_indptr[-1] valid),
    kv_last_page_len [rows] or None), the paged-KV CSR form of
    build_flashinfer_kv_indices (compact_attn/csrc/compactattn/cache_fill_kernel.cu:485-505)."""
    _need_cuda("table", table, torch.int32)
    _need_cuda("counts", counts, torch.int32)
    rows = batch * num_kv_heads
    if table.dim() != 2 or table.stride(1) != 1 or table.shape[0] < rows or table.shape[1] < kv_cap:
        raise ValueError("table must be [B*Hkv, >= kv_cap] with contiguous rows")
    if counts.numel() < rows:
        raise ValueError("counts must hold B*Hkv entries")
    d = make_dims(batch, BLOCK, num_kv_heads, num_kv_heads, kv_cap)
    dev = table.device
    indptr = torch.empty((rows + 1,), dtype=torch.int32, device=dev)
    indices = torch.empty((rows * kv_cap,), dtype=torch.int32, device=dev)
    last = torch.empty((rows,), dtype=torch.int32, device=dev) if with_last_page_len else None
    check(_hip.lib().ca_table_to_csr(ctypes.byref(d), table.data_ptr(), table.stride(0), counts.data_ptr(),
                                     indptr.data_ptr(), indices.data_ptr(), indices.numel(), _ptr(last), _stream()))
    return indptr, indices, last


def attn_workspace_bytes(past_blocks: Sequence[int], q_len: int, num_q_heads: int, num_kv_heads: int, kv_cap: int,
                         num_splits: int = 0) -> int:
    d = make_dims(len(past_blocks), q_len, num_q_heads, num_kv_heads, kv_cap)
    n = _hip.lib().ca_attn_workspace_size(ctypes.byref(d), past_array(past_blocks, d.batch), int(num_splits))
    if n < 0:
        raise _hip.CaError(int(n), _hip.last_error())
    return int(n)


def attn_pick_splits(past_blocks: Sequence[int], q_len: int, num_q_heads: int, num_kv_heads: int,
                     kv_cap: int) -> int:
    d = make_dims(len(past_blocks), q_len, num_q_heads, num_kv_heads, kv_cap)
    n = _hip.lib().ca_attn_pick_splits(ctypes.byref(d), past_array(past_blocks, d.batch))
    if n < 0:
        raise _hip.CaError(int(n), _hip.last_error())
    return int(n)


def attn_fwd(q: torch.Tensor, k: KV, v: KV, table: torch.Tensor, counts: torch.Tensor, past_blocks: Sequence[int],
             scale: float, kv_cap: int, num_kv_heads: int, out: Optional[torch.Tensor] = None, with_lse: bool = False,
             num_splits: int = 0, workspace: Optional[torch.Tensor] = None):
    """Indexed attention prefill; q/out [B, Lq, Hq, 128] bf16.  num_splits = 0 lets the
    library pick the split count; a positive value splits every row that many ways."""
    B, Lq, Hq, _ = q.shape
    ql = seq_layout(q, "q")
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape):
        raise ValueError(f"out {tuple(out.shape)} must have q's shape {tuple(q.shape)}")
    ol = seq_layout(out, "out")
    _need_cuda("table", table, torch.int32)
    _need_cuda("counts", counts, torch.int32)
    if table.dim() != 2 or table.stride(1) != 1 or table.shape[0] < B * num_kv_heads or table.shape[1] < kv_cap:
        raise ValueError("table must be [B*Hkv, >= kv_cap] with contiguous rows")
    if counts.numel() < B * num_kv_heads:
        raise ValueError("counts must hold B*Hkv entries")
    blocks = max(int(p) for p in past_blocks) + -(-Lq // BLOCK)  # blocks a row's table may name
    tokens = BLOCK * max(int(p) for p in past_blocks) + Lq  # reads stop at each request's 64 P + Lq
    for name, kv in (("k", k), ("v", v)):
        kv.check_blocks(name, B, num_kv_heads, blocks, tokens=tokens)
    d = make_dims(B, Lq, Hq, num_kv_heads, kv_cap)
    pa = past_array(past_blocks, d.batch)
    # num_splits = 0 hands the choice to the library
    need = _hip.lib().ca_attn_workspace_size(ctypes.byref(d), pa, int(num_splits))
    if need < 0:
        raise _hip.CaError(int(need), _hip.last_error())
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty((need,), dtype=torch.uint8, device=q.device)
    lse = torch.empty((B, Hq, Lq), dtype=torch.float32, device=q.device) if with_lse else None
    check(_hip.lib().ca_attn_fwd(ctypes.byref(d), ctypes.byref(ql), ctypes.byref(k.layout), ctypes.byref(v.layout),
                                 table.data_ptr(), table.stride(0), counts.data_ptr(), pa, float(scale),
                                 ctypes.byref(ol), _ptr(lse), int(num_splits), _ptr(workspace),
                                 int(need), _stream()))
    return (out, lse) if with_lse else out


def attn_decode_workspace_bytes(kv_len: Sequence[int], q_len: int, num_q_heads: int, num_kv_heads: int,
                                kv_cap: int, num_splits: int = 0) -> int:
    d = make_dims(len(kv_len), q_len, num_q_heads, num_kv_heads, kv_cap)
    n = _hip.lib().ca_attn_decode_workspace_size(ctypes.byref(d), past_array(kv_len, d.batch), int(num_splits))
    if n < 0:
        raise _hip.CaError(int(n), _hip.last_error())
    return int(n)


def attn_decode(q: torch.Tensor, k: KV, v: KV, kv_len: Sequence[int], scale: float, kv_cap: int, num_kv_heads: int,
                out: Optional[torch.Tensor] = None, with_lse: bool = False, num_splits: int = 0,
                workspace: Optional[torch.Tensor] = None):
    """Dense decode attention over the whole cache: q/out [B, q_len, Hq, 128] bf16 (q_len 1..64),
    the q_len rows being the last positions of each request's kv_len[b] tokens.

    Replaces the q_len == 1 branch of LlamaSeerAttentionChunkedDense.forward
    (compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:878-894)."""
    B, Lq, Hq, _ = q.shape
    if len(kv_len) != B:
        raise ValueError(f"kv_len has {len(kv_len)} entries for batch {B}")
    ql = seq_layout(q, "q")
    if out is None:
        out = torch.empty_like(q)
    elif tuple(out.shape) != tuple(q.shape):
        raise ValueError(f"out {tuple(out.shape)} must have q's shape {tuple(q.shape)}")
    ol = seq_layout(out, "out")
    # the kernel's buffer ranges end at each request's kv_len: a contiguous cache needs those
    # tokens only, a paged one a page for every block they touch
    max_len = max(int(x) for x in kv_len)
    for name, kv in (("k", k), ("v", v)):
        kv.check_blocks(name, B, num_kv_heads, (max_len + BLOCK - 1) // BLOCK, tokens=max_len)
    d = make_dims(B, Lq, Hq, num_kv_heads, kv_cap)
    ka = past_array(kv_len, d.batch)
    need = _hip.lib().ca_attn_decode_workspace_size(ctypes.byref(d), ka, int(num_splits))
    if need < 0:
        raise _hip.CaError(int(need), _hip.last_error())
    if need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty((need,), dtype=torch.uint8, device=q.device)
    lse = torch.empty((B, Hq, Lq), dtype=torch.float32, device=q.device) if with_lse else None
    check(_hip.lib().ca_attn_decode(ctypes.byref(d), ctypes.byref(ql), ctypes.byref(k.layout), ctypes.byref(v.layout),
                                    ka, float(scale), ctypes.byref(ol), _ptr(lse), int(num_splits),
                                    _ptr(workspace), int(need), _stream()))
    return (out, lse) if with_lse else out


# ----------------------------------------------------------------------------- model plumbing
def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(x * cos + rotate_half(x) * sin) for x [B, L, H, 128] bf16 and fp32 cos/sin [L, 128];
    bit-identical to apply_rotary_pos_emb evaluated in fp32."""
    B, L, H, _ = x.shape
    xl = seq_layout(x, "x")
    for name, t in (("cos", cos), ("sin", sin)):
        _need_cuda(name, t, torch.float32)
        if t.shape != (L, HEAD_DIM) or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous fp32 [{L}, {HEAD_DIM}]")
    if out is None:
        out = torch.empty((B, L, H, HEAD_DIM), dtype=torch.bfloat16, device=x.device)
    yl = seq_layout(out, "out")
    check(_hip.lib().ca_rope_apply(ctypes.byref(xl), ctypes.byref(yl), B, L, H, cos.data_ptr(), sin.data_ptr(),
                                   _stream()))
    return out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: Optional[torch.Tensor] = None):
    """bf16(w * bf16(x * rsqrt(mean(x^2) + eps))) over the last dim of a bf16 tensor.  With
    ``residual`` the norm is taken of s = bf16(x + residual) and (s, y) is returned."""
    _need_cuda("x", x, torch.bfloat16)
    _need_cuda("weight", weight, torch.bfloat16)
    n = x.shape[-1]
    if weight.shape != (n,) or not weight.is_contiguous() or x.stride(-1) != 1:
        raise ValueError("x needs a contiguous last dim and weight [n]")
    x2 = x.reshape(-1, n)
    out = torch.empty((x2.shape[0], n), dtype=torch.bfloat16, device=x.device)
    r_ptr = s_ptr = 0
    r2 = s2 = None
    if residual is not None:
        _need_cuda("residual", residual, torch.bfloat16)
        if residual.shape != x.shape or residual.stride(-1) != 1:
            raise ValueError("residual must match x's shape with a contiguous last dim")
        r2 = residual.reshape(-1, n)
        s2 = torch.empty_like(out)
        r_ptr, s_ptr = r2.data_ptr(), s2.data_ptr()
    check(_hip.lib().ca_rmsnorm(x2.data_ptr(), x2.stride(0), r_ptr, r2.stride(0) if r2 is not None else 0, s_ptr,
                                s2.stride(0) if s2 is not None else 0, weight.data_ptr(), out.data_ptr(),
                                out.stride(0), x2.shape[0], n, float(eps), _stream()))
    if residual is None:
        return out.view(x.shape)
    return s2.view(x.shape), out.view(x.shape)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """bf16(bf16(silu(gate)) * up) for bf16 tensors of one shape."""
    _need_cuda("gate", gate, torch.bfloat16)
    _need_cuda("up", up, torch.bfloat16)
    if gate.shape != up.shape or gate.stride(-1) != 1 or up.stride(-1) != 1:
        raise ValueError("gate and up must share a shape with contiguous last dims")
    n = gate.shape[-1]
    g2, u2 = gate.reshape(-1, n), up.reshape(-1, n)
    out = torch.empty((g2.shape[0], n), dtype=torch.bfloat16, device=gate.device)
    check(_hip.lib().ca_swiglu(g2.data_ptr(), g2.stride(0), u2.data_ptr(), u2.stride(0), out.data_ptr(), out.stride(0),
                               g2.shape[0], n, _stream()))
    return out.view(gate.shape)
