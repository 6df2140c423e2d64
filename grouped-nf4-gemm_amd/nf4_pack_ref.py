"""NF4 fixture packer in plain torch (no bitsandbytes).

Storage contract (reference kernel/nf4_pack_ref.py:20-57, the layout the
kernels read): a weight row is cut into 64-element blocks; a block's scale is
its largest magnitude (at least 1e-12, so an all-zero block still divides);
every element is stored as the index of the NF4 codebook value nearest to
element / scale, the lower index winning an exact tie; two indices share a
byte, the even element in the high nibble. The bytes are not claimed to be
those of bitsandbytes' quantizer: the kernels are checked against the decode
of whatever bytes this produces.
"""
from __future__ import annotations

import torch

from nf4_grouped import BLOCKSIZE, NF4_LUT

_SCALE_FLOOR = 1e-12


def nearest_code(x: torch.Tensor, table) -> torch.Tensor:
    """Index of the nearest ``table`` entry for every element of fp32 ``x``
    (uint8). One pass per entry with a strict comparison, so on an exact tie
    the lowest index stays: the same choice as an argmin over |x - table|
    evaluated in fp32, without a [..., 16] temporary."""
    entries = torch.tensor(table, dtype=torch.float32)
    best = torch.zeros(x.shape, dtype=torch.uint8, device=x.device)
    best_d = (x - entries[0]).abs()
    for i in range(1, len(table)):
        d = (x - entries[i]).abs()
        closer = d < best_d
        best = torch.where(closer, torch.tensor(i, dtype=torch.uint8, device=x.device), best)
        best_d = torch.minimum(best_d, d)
    return best


def quantize_pack_nf4(w: torch.Tensor):
    """``w [N, K]`` -> ``(packed [N, K/2] uint8, absmax [N, K/64] fp32)``.

    One expert at a time: a 3-D stack is refused (pack each expert, or use
    ``make_stack`` for synthetic stacks)."""
    if w.dim() != 2:
        raise ValueError(f"quantize_pack_nf4 packs one [N, K] expert weight, got shape "
                         f"{tuple(w.shape)}; pack experts one by one or call make_stack()")
    rows, cols = w.shape
    if cols % BLOCKSIZE:
        raise ValueError(f"K={cols} is not a multiple of the {BLOCKSIZE}-element block")
    x = w.to(torch.float32).reshape(rows, cols // BLOCKSIZE, BLOCKSIZE)
    scale = torch.clamp(x.abs().max(dim=-1).values, min=_SCALE_FLOOR)
    idx = nearest_code((x / scale.unsqueeze(-1)).reshape(rows, cols), NF4_LUT)
    pairs = idx.reshape(rows, cols // 2, 2)
    packed = (pairs[..., 0] << 4) | pairs[..., 1]      # even element: high nibble
    return packed.contiguous(), scale.contiguous()


def make_stack(E: int, N: int, K: int, seed: int = 0, device: str = "cpu", scale: float = 1.0):
    """``E`` seeded N(0, scale^2) experts, packed: ``(B [E, N, K/2] u8,
    absmax [E, N, K/64] f32)`` on ``device``."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    packed, absmax = zip(*(quantize_pack_nf4(torch.randn(N, K, generator=gen) * scale)
                           for _ in range(E)))
    return torch.stack(packed).to(device), torch.stack(absmax).to(device)
