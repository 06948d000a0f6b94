"""GPU tests of the fused element-wise kernels of the Llama integration (rotary embedding,
RMSNorm with and without the residual add, SwiGLU product) against fp32 PyTorch
references of the same formulas evaluated on the CPU.

- rotary: bit-identical to apply_rotary_pos_emb in fp32 (same operations, same order);
- RMSNorm / SwiGLU: within one bf16 ulp of the reference everywhere (the fp32 sum of
  squares and the exponential are this build's own, so a last-bit fp32 difference can move
  a bf16 rounding), and equal on all but a small fraction of elements; with a norm weight
  the one-ulp step of the normalised value is scaled by w before the final rounding, so
  the bound there is two ulps;
- the residual form returns exactly bf16(x + r) and exactly the plain norm of that sum.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from compactattention_amd import ops
from compactattention_amd.prefill_sparse.llama import SeerAttnLlamaConfig
from compactattention_amd.prefill_sparse.llama.modeling_llama_common import (LlamaRotaryEmbedding,
                                                                             apply_rotary_pos_emb)

from .util import bits

pytestmark = pytest.mark.gpu


def _ulps(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 tensors of one shape (+0 and -0 coincide)."""
    def key(t):
        v = bits(t).astype(np.int32)
        mag = v & 0x7FFF
        return np.where(v & 0x8000, -mag, mag)
    return np.abs(key(a) - key(b))


def _rotary(gpu, max_pos=8192):
    cfg = SeerAttnLlamaConfig(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=1,
                              num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=max_pos,
                              rope_theta=500000.0)
    return LlamaRotaryEmbedding(cfg, device=gpu)


@pytest.mark.parametrize("B,L,H,start", [(1, 64, 32, 0), (2, 192, 8, 4096), (3, 5, 2, 77), (1, 1, 4, 8000)])
def test_rope_bit_exact(gpu, B, L, H, start):
    print(f"case: rope B={B} L={L} H={H} start={start}", flush=True)
    rot = _rotary(gpu)
    cos, sin = rot.tokens(start, L)
    g = torch.Generator().manual_seed(B * 1000 + L)
    # x is a strided view (heads 1..H of a wider projection), as q/k views of a fused output
    wide = (torch.randn(B, L, H + 3, 128, generator=g) * 4).bfloat16().to(gpu)
    x = wide[:, :, 1:H + 1]
    got = ops.rope(x, cos, sin)
    ref, _ = apply_rotary_pos_emb(x.cpu(), x.cpu(), cos.cpu(), sin.cpu())
    assert np.array_equal(bits(got), bits(ref))
    # output into a strided destination
    dst = torch.zeros(B, L, H + 1, 128, dtype=torch.bfloat16, device=gpu)
    ops.rope(x, cos, sin, out=dst[:, :, 1:])
    assert np.array_equal(bits(dst[:, :, 1:]), bits(ref))
    assert not dst[:, :, 0].any()


def _rms_ref(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """transformers' LlamaRMSNorm on the CPU: fp32 statistics, bf16 normalised value times w."""
    xc = x.float().cpu()
    return w.cpu() * F.rms_norm(xc, (xc.shape[-1],), eps=eps).bfloat16()


@pytest.mark.parametrize("rows,n,pad", [(37, 4096, 0), (5, 256, 8), (3, 136, 16), (1024, 8192, 0), (2, 8, 0)])
def test_rmsnorm_matches_torch(gpu, rows, n, pad):
    print(f"case: rmsnorm rows={rows} n={n} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + n)
    x = (torch.randn(rows, n + pad, generator=g) * 3).bfloat16().to(gpu)[:, :n]
    ones = torch.ones(n, dtype=torch.bfloat16, device=gpu)
    d = _ulps(ops.rmsnorm(x, ones, 1e-5), _rms_ref(x, ones, 1e-5))
    assert d.max() <= 1, d.max()
    assert (d > 0).mean() < 1e-2, (d > 0).mean()
    w = (torch.rand(n, generator=g) + 0.5).bfloat16().to(gpu)
    d = _ulps(ops.rmsnorm(x, w, 1e-5), _rms_ref(x, w, 1e-5))
    assert d.max() <= 2, d.max()
    assert (d > 0).mean() < 1e-2, (d > 0).mean()


@pytest.mark.parametrize("rows,n", [(33, 4096), (4, 264)])
def test_rmsnorm_residual_form(gpu, rows, n):
    print(f"case: add+rmsnorm rows={rows} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows + n)
    x = (torch.randn(rows, n, generator=g) * 2).bfloat16().to(gpu)
    r = (torch.randn(rows, n, generator=g) * 5).bfloat16().to(gpu)
    w = (torch.rand(n, generator=g) + 0.5).bfloat16().to(gpu)
    s, y = ops.rmsnorm(x, w, 1e-6, residual=r)
    assert np.array_equal(bits(s), bits(x.cpu() + r.cpu()))  # bf16 add, rounded once
    assert np.array_equal(bits(y), bits(ops.rmsnorm(s, w, 1e-6)))
    d = _ulps(y, _rms_ref(s, w, 1e-6))
    assert d.max() <= 2


@pytest.mark.parametrize("rows,n", [(19, 14336), (256, 512), (3, 8)])
def test_swiglu_matches_torch(gpu, rows, n):
    print(f"case: swiglu rows={rows} n={n}", flush=True)
    g = torch.Generator().manual_seed(rows * 3 + n)
    gu = (torch.randn(rows, 2 * n, generator=g) * 4).bfloat16().to(gpu)
    gate, up = gu[:, :n], gu[:, n:]  # strided halves of one projection output
    got = ops.swiglu(gate, up)
    ref = F.silu(gate.float().cpu()).bfloat16() * up.cpu()
    d = _ulps(got, ref)
    assert d.max() <= 1, d.max()
    assert (d > 0).mean() < 1e-2, (d > 0).mean()
    # the extremes: silu saturates to g for large g and to -0 for very negative g
    ext = torch.tensor([[-200.0, -90.0, -20.0, -1e-3, 0.0, 1e-3, 20.0, 90.0]], dtype=torch.bfloat16).to(gpu)
    one = torch.ones_like(ext)
    got_e = ops.swiglu(ext, one)
    ref_e = F.silu(ext.float().cpu()).bfloat16()
    assert _ulps(got_e, ref_e).max() <= 1
