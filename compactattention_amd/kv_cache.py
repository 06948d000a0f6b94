"""Paged KV cache owned by the compactattn path: a page pool, a page table and an allocator.

Replaces transformers' DynamicCache concatenation for the chunked-prefill layers
(compact_attn/prefill_sparse/llama/modeling_llama_seerattn_chunked_dense.py:518-536 and the
heads-first _hf cache, modeling_llama_seerattn_chunked_dense_hf.py:59-82), the grow-only page
workspaces of the reference's paged prefill (compact_attn/kernels/varlen/
indexed_dense_prefill_varlen.py:190-463), the per-layer mean-K cache of the FlashPrefill
model (modeling_llama_flashprefill_compactattn.py:121-150) and the gate K-block cache of the
Seer model (modeling_llama_seerattn_chunked_dense.py:398-478).

Layout of one layer:
  - K and V pages: a pool of 64-token pages ``[num_pages, 64, 128]`` bf16 each (one 16 KiB
    page per (request, KV head, logical block)); the pool only grows, and growing keeps every
    page id (the contents move to the larger pool once);
  - the page table: int32 ``[B*Hkv, blocks]`` (row = b*Hkv + h), logical block -> page id,
    kept on the device for the kernels and mirrored on the host, where pages are allocated;
  - block summaries by logical block: kmean ``[B, Hkv, blocks, 128]`` fp32 (FlashPrefill
    scoring) and, with a gate, kgate ``[B, gate_heads, blocks, 128]`` fp32.  ``kmean_blocks`` /
    ``kgate_blocks`` count the leading blocks whose summaries are valid: decode appends write
    no summaries, so a block that decode tokens complete has none until the next chunk append
    recomputes its mean-K from the cached keys (the reference's FlashPrefill model recomputes
    its mean-K cache when the token count disagrees, modeling_llama_flashprefill_compactattn.py:
    128-147).  Gate-K summaries come from pre-RoPE keys the cache does not hold, so a chunk that
    follows such a block raises (``require_kgate``).
Pages are reference-counted: ``fork`` lets a request share another's pages, and a decode
append into a shared, partly filled page copies it first.  Appends write the chunk's pages
and summaries in place through the cache-fill kernel; nothing is ever re-copied.

Host-side allocation happens in ``append``/``append_tokens`` before the kernels are launched
(a small page-table upload on the current stream), so a HIP graph that captures the chunk
step must be recorded after the cache holds its pages (``reserve``).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np
import torch

from . import ops

BLOCK = 64
HEAD_DIM = 128


class PagePool:
    """Grow-only pool of 64-token K and V pages with reference counts."""

    def __init__(self, num_pages: int, device):
        num_pages = max(int(num_pages), 1)
        self.device = torch.device(device)
        self.k = torch.zeros((num_pages, BLOCK, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
        self.v = torch.zeros_like(self.k)
        self.refs = np.zeros(num_pages, np.int32)
        self._free: List[int] = list(range(num_pages - 1, -1, -1))  # pop() hands out ascending ids

    @property
    def num_pages(self) -> int:
        return self.k.shape[0]

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def alloc(self, n: int) -> List[int]:
        """n fresh pages (reference count 1); the pool grows (at least doubling) when short."""
        if n > len(self._free):
            self._grow(n - len(self._free))
        pages = [self._free.pop() for _ in range(n)]
        self.refs[pages] = 1
        return pages

    def retain(self, pages) -> None:
        np.add.at(self.refs, np.asarray(pages, np.int64), 1)

    def release(self, pages) -> None:
        for p in np.asarray(pages, np.int64).ravel().tolist():
            if self.refs[p] <= 0:
                raise RuntimeError(f"page {p} released more often than it was taken")
            self.refs[p] -= 1
            if self.refs[p] == 0:
                self._free.append(p)

    def _grow(self, need: int) -> None:
        old = self.num_pages
        new = max(2 * old, old + need)
        for name in ("k", "v"):
            t = torch.zeros((new, BLOCK, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
            t[:old].copy_(getattr(self, name))
            setattr(self, name, t)
        self.refs = np.concatenate([self.refs, np.zeros(new - old, np.int32)])
        self._free = list(range(new - 1, old - 1, -1)) + self._free


class PagedKVCache:
    """One layer's paged K/V cache for ``batch`` requests that advance together."""

    def __init__(self, batch: int, num_kv_heads: int, max_tokens: int, device, with_kmean: bool = True,
                 with_kgate: bool = False, kgate_heads: Optional[int] = None, pool_pages: Optional[int] = None):
        """max_tokens sizes the page table and summaries (they grow on demand); pool_pages
        sizes the initial page pool (default: every row's max_tokens)."""
        self.batch = batch
        self.num_kv_heads = num_kv_heads
        self.rows = batch * num_kv_heads
        self.device = torch.device(device)
        self.cap = max(-(-int(max_tokens) // BLOCK), 1)  # blocks per row of the table and summaries
        self.pool = PagePool(pool_pages if pool_pages is not None else self.rows * self.cap, self.device)
        self._pt = np.full((self.rows, self.cap), -1, np.int32)  # host mirror; -1 = unmapped
        self.page_table = torch.full((self.rows, self.cap), -1, dtype=torch.int32, device=self.device)
        self.kgate_heads = kgate_heads or num_kv_heads
        self.kmean = self._summary(num_kv_heads) if with_kmean else None
        self.kgate = self._summary(self.kgate_heads) if with_kgate else None
        self.length = 0  # tokens stored per request
        self.kmean_blocks = 0  # leading blocks with a valid kmean
        self.kgate_blocks = 0  # leading blocks with a valid kgate

    # -- layout ---------------------------------------------------------------------------
    def _summary(self, heads: int) -> torch.Tensor:
        return torch.zeros((self.batch, heads, self.cap, HEAD_DIM), dtype=torch.float32, device=self.device)

    @property
    def past_blocks(self) -> int:
        return self.length // BLOCK

    def layouts(self) -> Tuple[ops.KV, ops.KV]:
        """K and V as (pool, page table) layouts for the kernels."""
        return ops.KV.paged(self.pool.k, self.page_table), ops.KV.paged(self.pool.v, self.page_table)

    def pages_of(self, b: int, h: int) -> List[int]:
        """Page ids of request b, KV head h, in logical block order (the mapped blocks)."""
        row = self._pt[b * self.num_kv_heads + h]
        return row[row >= 0].tolist()

    # -- allocation -----------------------------------------------------------------------
    def _grow_cap(self, blocks: int) -> None:
        if blocks <= self.cap:
            return
        new = max(2 * self.cap, blocks)
        pt = np.full((self.rows, new), -1, np.int32)
        pt[:, :self.cap] = self._pt
        self._pt = pt
        dev_pt = torch.full((self.rows, new), -1, dtype=torch.int32, device=self.device)
        dev_pt[:, :self.cap].copy_(self.page_table)
        self.page_table = dev_pt
        for name in ("kmean", "kgate"):
            old = getattr(self, name)
            if old is not None:
                t = torch.zeros((old.shape[0], old.shape[1], new, HEAD_DIM), dtype=torch.float32, device=self.device)
                t[:, :, :self.cap].copy_(old)
                setattr(self, name, t)
        self.cap = new

    def _upload(self, b0: int, b1: int) -> None:
        if b1 > b0:
            self.page_table[:, b0:b1].copy_(torch.from_numpy(np.ascontiguousarray(self._pt[:, b0:b1])))

    def _map(self, b0: int, b1: int) -> None:
        """Give every row a page for each unmapped logical block in [b0, b1)."""
        self._grow_cap(b1)
        need = self._pt[:, b0:b1] < 0
        n = int(need.sum())
        if n:  # only new pages touch the device table (a small upload on the current stream)
            pages = np.asarray(self.pool.alloc(n), np.int32)
            block = self._pt[:, b0:b1]
            block[need] = pages  # row-major: a row's new blocks get ascending page ids
            self._pt[:, b0:b1] = block
            self._upload(b0, b1)

    def reserve(self, tokens: int) -> None:
        """Map pages for the first ``tokens`` tokens of every request ahead of time."""
        self._map(0, -(-int(tokens) // BLOCK))

    def _unshare(self, kb: int) -> None:
        """Copy-on-write of logical block kb: rows (in order) whose page still has other holders
        move to a copy; the last holder of a page keeps it."""
        col = self._pt[:, kb]
        refs = {int(p): int(self.pool.refs[p]) for p in col if p >= 0}
        moved = []
        for r in range(self.rows):
            p = int(col[r])
            if p >= 0 and refs[p] > 1:
                refs[p] -= 1
                moved.append(r)
        if not moved:
            return
        old = [int(col[r]) for r in moved]
        fresh = self.pool.alloc(len(moved))
        src = torch.as_tensor(old, device=self.device, dtype=torch.long)
        dst = torch.as_tensor(fresh, device=self.device, dtype=torch.long)
        self.pool.k[dst] = self.pool.k[src]
        self.pool.v[dst] = self.pool.v[src]
        self.pool.release(old)
        for r, p in zip(moved, fresh):
            self._pt[r, kb] = p
        self._upload(kb, kb + 1)

    # -- appends --------------------------------------------------------------------------
    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, gate_wk: Optional[torch.Tensor] = None,
               rope_cos: Optional[torch.Tensor] = None, rope_sin: Optional[torch.Tensor] = None) -> int:
        """Append a chunk of [B, L, Hkv, 128] bf16 K/V at a block boundary through the cache-fill
        kernel, which also writes the new blocks' kmean (and, with gate_wk [Hkv, 128, 128], the
        avg-pooled gate-K summaries); returns the number of past blocks before the append.  When
        L is not a multiple of 64 the last block holds L % 64 tokens: its summaries pool those
        (a kgate one stays valid, as the reference's gate cache keeps it; a kmean one is
        recomputed once decode tokens complete the block)."""
        B, L, Hkv, _ = k_new.shape
        if B != self.batch or Hkv != self.num_kv_heads:
            raise ValueError("k_new does not match the cache's batch / KV heads")
        if L < 1:
            raise ValueError("appended chunks hold at least one token")
        if self.length % BLOCK:
            raise ValueError("chunked prefill cannot follow decode steps that left a partial block")
        if gate_wk is not None and (self.kgate is None or self.kgate_heads != Hkv):
            raise ValueError("cache built without a per-KV-head gate-K summary buffer")
        past = self.past_blocks
        if gate_wk is not None:
            self.require_kgate(past)
        self.refresh_kmean(past)
        self._map(past, past - (-L // BLOCK))
        K, V = self.layouts()
        ops.cache_fill(k_new, v_new, K, V, [past] * B, self.cap, self.kmean, gate_wk=gate_wk, rope_cos=rope_cos,
                       rope_sin=rope_sin, kgate=self.kgate if gate_wk is not None else None)
        self.length += L
        if self.kmean is not None:
            self.kmean_blocks = self.past_blocks
        if gate_wk is not None:
            self.kgate_blocks = -(-self.length // BLOCK)
        return past

    def append_with_query_means(self, k_new: torch.Tensor, v_new: torch.Tensor,
                                q: torch.Tensor) -> Tuple[int, torch.Tensor]:
        """append(k_new, v_new) and the chunk's query-block means ([B, L, Hq, 128] bf16 ->
        qhat [B, Hq, ceil(L/64), 128] fp32, the FlashPrefill pooled queries) in one kernel launch;
        returns (past blocks before the append, qhat)."""
        B, L, Hkv, _ = k_new.shape
        if B != self.batch or Hkv != self.num_kv_heads:
            raise ValueError("k_new does not match the cache's batch / KV heads")
        if L < 1:
            raise ValueError("appended chunks hold at least one token")
        if self.length % BLOCK:
            raise ValueError("chunked prefill cannot follow decode steps that left a partial block")
        if self.kmean is None:
            raise ValueError("cache built without the mean-K summaries")
        past = self.past_blocks
        self.refresh_kmean(past)
        self._map(past, past - (-L // BLOCK))
        K, V = self.layouts()
        qhat = ops.cache_fill_pool_query(k_new, v_new, K, V, [past] * B, self.cap, self.kmean, q)
        self.length += L
        self.kmean_blocks = self.past_blocks
        return past, qhat

    def refresh_kmean(self, upto: int) -> None:
        """Write the mean-K of blocks [kmean_blocks, upto) from the cached keys (blocks that
        decode appends completed), by the cache-fill kernel in summaries-only mode; the means
        are the ones a chunk append of the same keys writes, bit for bit."""
        if self.kmean is None or self.kmean_blocks >= upto:
            return
        b0 = self.kmean_blocks
        idx = torch.from_numpy(np.ascontiguousarray(self._pt[:, b0:upto]).astype(np.int64)).to(self.device)
        n = (upto - b0) * BLOCK
        keys = self.pool.k[idx.reshape(-1)].view(self.batch, self.num_kv_heads, n, HEAD_DIM).transpose(1, 2)
        ops.cache_fill(keys, None, None, None, [b0] * self.batch, self.cap, self.kmean)
        self.kmean_blocks = upto

    def require_kgate(self, past: int) -> None:
        """A selecting chunk at ``past`` blocks needs gate-K summaries for every past block."""
        if self.kgate is not None and self.kgate_blocks < past:
            raise ValueError(f"gate-K summaries are missing for blocks [{self.kgate_blocks}, {past}): decode tokens "
                             "completed them and the cache keeps no pre-RoPE keys to pool; prefill the rest of the "
                             "sequence densely or start it again")

    def append_tokens(self, k_new: torch.Tensor, v_new: torch.Tensor) -> int:
        """Decode append: [B, L, Hkv, 128] bf16 K/V (any L) at the current length, which need
        not be block-aligned; returns the length before the append.  Block summaries are
        not maintained for these tokens, so chunked prefill cannot follow decode steps
        (append() rejects a length that is not a multiple of 64)."""
        B, L, Hkv, _ = k_new.shape
        if B != self.batch or Hkv != self.num_kv_heads:
            raise ValueError("k_new does not match the cache's batch / KV heads")
        if L == 0:
            return self.length
        start = self.length
        end = start + L
        self._map(start // BLOCK, -(-end // BLOCK))
        if start % BLOCK:
            self._unshare(start // BLOCK)
        pos = np.arange(start, end)
        pages = self._pt[:, pos // BLOCK].astype(np.int64)  # [rows, L]
        flat = torch.from_numpy(pages * BLOCK + (pos % BLOCK)[None, :]).to(self.device)
        kf = self.pool.k.view(-1, HEAD_DIM)
        vf = self.pool.v.view(-1, HEAD_DIM)
        kf[flat.reshape(-1)] = k_new.transpose(1, 2).reshape(-1, HEAD_DIM)
        vf[flat.reshape(-1)] = v_new.transpose(1, 2).reshape(-1, HEAD_DIM)
        self.length = end
        return start

    # -- sharing --------------------------------------------------------------------------
    def fork(self, src: int, dst: int) -> None:
        """Request dst takes request src's contents by sharing its pages (no copy): dst's own
        pages are released, src's gain a reference, and the summaries of src are copied."""
        if src == dst:
            return
        nb = -(-self.length // BLOCK)
        H = self.num_kv_heads
        for h in range(H):
            rs, rd = src * H + h, dst * H + h
            old = self._pt[rd][self._pt[rd] >= 0]
            self.pool.release(old)
            self._pt[rd] = -1
            self._pt[rd, :nb] = self._pt[rs, :nb]
            self.pool.retain(self._pt[rs, :nb])
        self._upload(0, self.cap)
        for t in (self.kmean, self.kgate):
            if t is not None:
                t[dst].copy_(t[src])

    # -- views ----------------------------------------------------------------------------
    def _gather(self, pool: torch.Tensor) -> torch.Tensor:
        nb = -(-self.length // BLOCK)
        idx = torch.from_numpy(self._pt[:, :nb].astype(np.int64)).to(self.device)
        pages = pool[idx.reshape(-1)].view(self.batch, self.num_kv_heads, nb * BLOCK, HEAD_DIM)
        return pages[:, :, :self.length]

    def k_hf(self) -> torch.Tensor:
        """The stored keys as a heads-first [B, Hkv, length, 128] tensor (a gathered copy)."""
        return self._gather(self.pool.k)

    def v_hf(self) -> torch.Tensor:
        return self._gather(self.pool.v)

    def reset(self, keep_pages: bool = False) -> None:
        """Empty the cache.  By default every request's pages go back to the pool (which keeps
        its size); with keep_pages the pages a row owns alone stay mapped for the next
        sequence (no allocation or page-table upload when it refills them), while pages
        shared with another request are released so a refill never writes into them."""
        if keep_pages:
            mapped = self._pt >= 0
            shared = mapped & (self.pool.refs[np.where(mapped, self._pt, 0)] > 1)
            if shared.any():
                self.pool.release(self._pt[shared])
                self._pt[shared] = -1
                self._upload(0, self.cap)
        else:
            mapped = self._pt[self._pt >= 0]
            if mapped.size:
                self.pool.release(mapped)
            self._pt[:] = -1
            self.page_table.fill_(-1)
        self.length = 0
        self.kmean_blocks = 0
        self.kgate_blocks = 0
