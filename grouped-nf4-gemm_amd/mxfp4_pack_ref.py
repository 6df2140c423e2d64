"""MXFP4 (e2m1 elements, e8m0 block scales) decode and fixture packer in
plain torch.

Format contract (reference kernel/mxfp4_pack_ref.py:21-103 and
kernel/mxfp4_grouped.py:34-37, the layout the kernels read):
  * ``FP4_VALUES``: the e2m1 codebook, index = sign << 3 | magnitude;
  * 32-element blocks, one e8m0 byte each: scale 2^(byte - 127);
  * two elements per byte, the even element in the LOW nibble;
  * checkpoint layout ``blocks [..., K/32, 16]`` and ``scales [..., K/32]``;
    flattened, ``blocks`` is the ``[..., K/2]`` array the kernels take.
``dequant_mxfp4`` scales exactly, like C's ldexp: byte 0xFF gives +-inf for
nonzero codes and keeps zeros at zero; byte 0x00 gives subnormals.
"""
from __future__ import annotations

import torch

from nf4_pack_ref import nearest_code

FP4_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
MX_BLOCK = 32
E8M0_BIAS = 127
E8M0_NAN = 0xFF
NIBBLE_LOW_FIRST = True

_FP4_TOP = 6.0            # largest e2m1 magnitude
_AMAX_FLOOR = 1e-20


def _lut(device, dtype=torch.float32):
    return torch.tensor(FP4_VALUES, dtype=dtype, device=device)


def dequant_mxfp4(blocks: torch.Tensor, scales: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """``blocks [..., n, 16]`` u8 and ``scales [..., n]`` u8 -> ``[..., n * 32]``."""
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("dequant_mxfp4 takes uint8 blocks and uint8 e8m0 scales")
    if blocks.shape[-1] != 16 or tuple(blocks.shape[:-1]) != tuple(scales.shape):
        raise ValueError(f"blocks {tuple(blocks.shape)} must be scales {tuple(scales.shape)} "
                         "plus a trailing 16")
    b = blocks.to(torch.int64)
    even, odd = (b & 0xF, b >> 4) if NIBBLE_LOW_FIRST else (b >> 4, b & 0xF)
    idx = torch.stack((even, odd), dim=-1).flatten(-2)           # [..., n, 32]
    vals = _lut(blocks.device, torch.float64)[idx]
    # 2^(s - 127) in float64 is finite for every byte, and every e2m1 value
    # times it is exact there: the one rounding is the final cast (inf for
    # 2^128 times a nonzero code, 0 for a zero code)
    step = torch.pow(torch.tensor(2.0, dtype=torch.float64, device=blocks.device),
                     scales.to(torch.float64) - E8M0_BIAS)
    return (vals * step.unsqueeze(-1)).to(dtype).flatten(-2)


def quantize_pack_mxfp4(w: torch.Tensor):
    """``w [..., K]`` -> ``(blocks [..., K/32, 16] u8, scales [..., K/32] u8)``.

    A block's exponent is ceil(log2(amax / 6)), kept within +-127, so its
    largest magnitude lands at the top of the e2m1 range; each scaled
    element stores its nearest codebook index (lowest index on a tie)."""
    *lead, cols = w.shape
    if cols % MX_BLOCK:
        raise ValueError(f"K={cols} is not a multiple of the {MX_BLOCK}-element block")
    x = w.to(torch.float32).reshape(*lead, cols // MX_BLOCK, MX_BLOCK)
    amax = torch.clamp(x.abs().max(dim=-1).values, min=_AMAX_FLOOR)
    expo = torch.clamp(torch.ceil(torch.log2(amax / _FP4_TOP)), -E8M0_BIAS, E8M0_BIAS)
    idx = nearest_code(x / torch.exp2(expo).unsqueeze(-1), FP4_VALUES)
    pairs = idx.reshape(*lead, cols // MX_BLOCK, MX_BLOCK // 2, 2)
    lo, hi = (pairs[..., 0], pairs[..., 1]) if NIBBLE_LOW_FIRST else (pairs[..., 1], pairs[..., 0])
    return (lo | (hi << 4)).contiguous(), (expo + E8M0_BIAS).to(torch.uint8).contiguous()
