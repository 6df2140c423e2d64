"""Pure-torch NF4 packer -- fixture generation without bitsandbytes.

Same storage semantics as the reference's packer (kernel/nf4_pack_ref.py:20-57):
per 64-element K block absmax = max|w| (clamped to >= 1e-12); each element
takes the nearest NF4 codebook entry of w / absmax (first index on ties);
element 2j goes to the HIGH nibble of byte j, 2j+1 to the LOW nibble. Not
claimed bit-identical to bitsandbytes' quantizer; the kernels are checked
against the decode of whatever bytes these produce.
"""
from __future__ import annotations

import torch

from nf4_grouped import BLOCKSIZE, NF4_LUT


def quantize_pack_nf4(w: torch.Tensor):
    """w [N, K] float -> (packed [N, K//2] uint8, absmax [N, K//64] fp32)."""
    if w.dim() != 2:
        raise ValueError(
            f"expected 2-D [N, K] per-expert weight; got shape {tuple(w.shape)} -- "
            "pack per expert and stack, or use make_stack() for synthetic fixtures.")
    N, K = w.shape
    assert K % BLOCKSIZE == 0, f"K={K} must be a multiple of {BLOCKSIZE}"
    lut = torch.tensor(NF4_LUT, dtype=torch.float32, device=w.device)
    blocks = w.float().reshape(N, K // BLOCKSIZE, BLOCKSIZE)
    absmax = blocks.abs().amax(dim=2).clamp_min(1e-12)
    scaled = (blocks / absmax[:, :, None]).reshape(N, K)
    # nearest codebook entry, first index on ties (argmin of |x - lut|),
    # evaluated in row chunks to bound the [rows, K, 16] temporary
    codes = torch.empty(N, K, dtype=torch.uint8, device=w.device)
    step = max(1, (1 << 22) // max(K, 1))
    for r in range(0, N, step):
        d = (scaled[r:r + step, :, None] - lut).abs()
        codes[r:r + step] = d.argmin(dim=2).to(torch.uint8)
    packed = (codes[:, 0::2] << 4) | codes[:, 1::2]
    return packed.contiguous(), absmax.to(torch.float32).contiguous()


def make_stack(E: int, N: int, K: int, seed: int = 0, device: str = "cpu", scale: float = 1.0):
    """E experts of seeded N(0, scale) weights -> (B [E,N,K/2] u8, absmax [E,N,K/64] f32)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    B = torch.empty(E, N, K // 2, dtype=torch.uint8)
    A = torch.empty(E, N, K // BLOCKSIZE, dtype=torch.float32)
    for e in range(E):
        w = torch.randn(N, K, generator=g, dtype=torch.float32) * scale
        B[e], A[e] = quantize_pack_nf4(w)
    return B.to(device), A.to(device)
