"""Pure-torch MXFP4 (e2m1 element, e8m0 scale) reference decode and packer.

Same semantics as the reference's module (kernel/mxfp4_pack_ref.py:21-103):
the e2m1 codebook FP4_VALUES (index = sign << 3 | magnitude), 32-element
blocks, e8m0 bias 127, element 2j in the LOW nibble. ``dequant_mxfp4``
applies the scale with ldexp, so a 0xFF scale gives +-inf for nonzero codes
and keeps zeros at zero. The checkpoint layout is ``blocks [..., K/32, 16]``
and ``scales [..., K/32]``; flattened, ``blocks`` is the [..., K/2] array the
kernels take.
"""
from __future__ import annotations

import torch

FP4_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
MX_BLOCK = 32
E8M0_BIAS = 127
E8M0_NAN = 0xFF
NIBBLE_LOW_FIRST = True


def _lut(device, dtype=torch.float32):
    return torch.tensor(FP4_VALUES, dtype=dtype, device=device)


def dequant_mxfp4(blocks: torch.Tensor, scales: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """blocks [..., n_blk, 16] u8, scales [..., n_blk] u8 -> [..., n_blk * 32]."""
    assert blocks.dtype == torch.uint8 and scales.dtype == torch.uint8
    assert blocks.shape[-1] == 16 and blocks.shape[:-1] == scales.shape, (blocks.shape, scales.shape)
    lut = _lut(blocks.device, dtype)
    lo = (blocks & 0x0F).long()
    hi = (blocks >> 4).long()
    first, second = (lo, hi) if NIBBLE_LOW_FIRST else (hi, lo)
    codes = torch.stack([first, second], dim=-1).reshape(*blocks.shape[:-1], 32)
    vals = lut[codes]
    exp = (scales.to(torch.int32) - E8M0_BIAS)[..., None]
    out = torch.ldexp(vals, exp)
    return out.reshape(*blocks.shape[:-2], blocks.shape[-2] * 32)


def quantize_pack_mxfp4(w: torch.Tensor):
    """w [..., K] float -> (blocks [..., K//32, 16] u8, scales [..., K//32] u8).

    Per 32-block the exponent e = ceil(log2(amax / 6)) (clamped to +-127)
    puts max|w| at the top of e2m1's range; each scaled element takes the
    nearest codebook entry (first index on ties)."""
    *lead, K = w.shape
    assert K % MX_BLOCK == 0, f"K={K} must be a multiple of {MX_BLOCK}"
    nb = K // MX_BLOCK
    wb = w.float().reshape(*lead, nb, MX_BLOCK)
    amax = wb.abs().amax(dim=-1).clamp_min(1e-20)
    e = torch.ceil(torch.log2(amax / 6.0)).clamp(-E8M0_BIAS, E8M0_BIAS)
    scaled = wb / torch.exp2(e)[..., None]
    lut = _lut(w.device)
    flat = scaled.reshape(-1, MX_BLOCK)
    codes = torch.empty(flat.shape, dtype=torch.uint8, device=w.device)
    step = 1 << 16
    for r in range(0, flat.shape[0], step):
        codes[r:r + step] = (flat[r:r + step, :, None] - lut).abs().argmin(dim=-1).to(torch.uint8)
    codes = codes.reshape(*lead, nb, MX_BLOCK)
    first, second = codes[..., 0::2], codes[..., 1::2]
    packed = (second << 4) | first if NIBBLE_LOW_FIRST else (first << 4) | second
    return packed.contiguous(), (e + E8M0_BIAS).to(torch.uint8).contiguous()
