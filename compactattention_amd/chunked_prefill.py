"""Chunked prefill driver for the compactattn models.

Restates run_chunked_prefill_once (eval/chunked_prefill/chunked_prefill_runtime.py:1103-1215)
for this path: the prompt is cut into chunk_size-token segments, each segment is one model
call over the shared per-layer cache with logits_to_keep=1; the first segment runs dense
(no past), every later one selects blocks.  Returns the last segment's logits and the
wall time of the whole prefill (device synchronised on both sides).
"""
from __future__ import annotations

import time
from typing import Optional, Tuple

import torch

from .prefill_sparse.llama.modeling_llama_common import ChunkedPrefillCache


@torch.no_grad()
def run_chunked_prefill_once(model: torch.nn.Module, input_ids: torch.Tensor, chunk_size: int,
                             cache: Optional[ChunkedPrefillCache] = None) -> Tuple[torch.Tensor, float]:
    B, T = input_ids.shape
    if chunk_size <= 0 or chunk_size % 64:
        raise ValueError("chunk_size must be a positive multiple of 64")
    # a prompt of any length: a final chunk that is not a multiple of 64 tokens selects with a
    # partial last block
    # a stock transformers model whose attention was replaced (load_attention_replacement)
    # takes the cache as past_key_values and returns a model output
    hf = getattr(getattr(model, "config", None), "seerattn_attention_harness", None) == "replacement"
    if cache is None:
        if hf:
            from .load_attention_replacement import new_compactattn_cache

            cache = new_compactattn_cache(model, B, T)
        else:
            cache = model.new_cache(B, T)
    else:
        cache.reset()
    logits = None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for start in range(0, T, chunk_size):
        end = min(start + chunk_size, T)
        if hf:
            logits = model(input_ids=input_ids[:, start:end], past_key_values=cache, use_cache=True,
                           logits_to_keep=1).logits
        else:
            logits = model(input_ids[:, start:end], cache, logits_to_keep=1)
    torch.cuda.synchronize()
    return logits, time.perf_counter() - t0


def synthetic_prompt(batch: int, tokens: int, vocab_size: int, seed: int, device) -> torch.Tensor:
    """Token ids drawn with torch.randint from one seeded generator (the reference harness
    draws its synthetic prompts the same way, chunked_prefill_runtime.py:588-599)."""
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randint(0, vocab_size, (batch, tokens), generator=g).to(device)
