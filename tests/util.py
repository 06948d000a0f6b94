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
