"""Grouped W4A16 GEMM over native MXFP4 expert stacks on MI355X (gfx950).

Drop-in for the reference module of the same name (kernel/mxfp4_grouped.py):
``gemm_mxfp4_grouped`` computes ``out[t] = a[t] @ dequant_mxfp4(W[e(t)]).T``
for tokens grouped by expert, in one launch, from ``blocks [E, N, K/2]`` uint8
(element 2j in the LOW nibble) and ``scales [E, N, K/32]`` uint8 e8m0.

Decode is one CDNA4 instruction per nibble pair (v_cvt_scalef32_pk_bf16_fp4:
e2m1 value times 2^(e-127) into bf16), which is exact for every finite scale,
so the only rounding in the op is the fp32 MFMA accumulation and the bf16
output. An e8m0 byte of 0xFF decodes as 2^128 = +inf (zero codes give NaN),
the exp2-multiply behaviour the reference allows on the GPU
(kernel/mxfp4_grouped.py:13-15); the CPU oracle keeps ldexp semantics.

``dgrad_mxfp4_grouped`` is the backward w.r.t. activations. The reference
has no GPU kernel for it (its backward loops experts in Python,
kernel/mxfp4_qlora.py:106-122); its CPU spec is gnf4_dgrad_mxfp4_grouped.
"""
from __future__ import annotations

import torch

import _hiplib
from nf4_grouped import (  # noqa: F401  (re-exported like the reference)
    _DGRAD_DEFAULT,
    _launch_dgrad,
    _launch_fwd,
    _prefill_block_m,
    _require_gpu,
    build_group_tiles,
)

# e2m1 codebook, index = sign << 3 | magnitude (reference kernel/mxfp4_grouped.py:34-37).
FP4_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
MX_BLOCK = 32
E8M0_BIAS = 127

_LUT_CACHE: dict = {}


def _lut(device):
    key = str(device)
    if key not in _LUT_CACHE:
        _LUT_CACHE[key] = torch.tensor(FP4_VALUES, dtype=torch.float32, device=device)
    return _LUT_CACHE[key]


def _flat_blocks(blocks):
    """Accept the checkpoint's [E, N, K/32, 16] layout as well as [E, N, K/2]."""
    if blocks.dim() == 4:
        E, N, nb, sixteen = blocks.shape
        assert sixteen == 16, blocks.shape
        return blocks.reshape(E, N, nb * 16)
    return blocks


def gemm_mxfp4_grouped(a_cat, blocks, scales, sizes, expert_ids,
                       block_m: int | None = None, prefill_variant: int | None = None):
    """Single-launch grouped MXFP4 GEMM (reference kernel/mxfp4_grouped.py:134-172).

    ``a_cat [T, K]`` bf16 (fp16 and fp32 are rounded to bf16 first),
    group-sorted; ``blocks [E, N, K//2]`` uint8;
    ``scales [E, N, K//32]`` uint8 e8m0; ``sizes`` per-group row counts;
    ``expert_ids [G]`` list / CPU tensor / device tensor. Returns ``[T, N]``
    bf16 in the same group order. Groups of <= 16 rows take the decode kernel
    (each expert's weights streamed once); larger groups the tiled MFMA
    kernel (``block_m`` forces it). ``prefill_variant`` is accepted (0, 1, 3)
    and does not change the result: e2m1 x 2^(e - 127) is exact in bf16, so
    every variant's weights (the reference's fp32 products of VARIANT 1
    included) are the same values."""
    blocks = _flat_blocks(blocks)
    E, N, _ = blocks.shape
    T, K = a_cat.shape
    assert sum(int(m) for m in sizes) == T, (sum(int(m) for m in sizes), T)
    assert tuple(scales.shape) == (E, N, K // MX_BLOCK), (tuple(scales.shape), (E, N, K // MX_BLOCK))
    assert blocks.dtype == torch.uint8 and scales.dtype == torch.uint8
    _require_gpu(
        a_cat, "gemm_mxfp4_grouped",
        "For a CPU-checkable decode of the same bytes use the pure-torch "
        "dequant_mxfp4 (mxfp4_pack_ref) or, for NF4 stacks, dequant_ref.")
    if K % MX_BLOCK or blocks.shape[2] * 2 != K:
        raise ValueError(f"K={K} must equal 2*blocks.shape[2] and be a multiple of {MX_BLOCK}")
    if prefill_variant is not None and prefill_variant not in (0, 1, 3):
        raise ValueError(f"prefill_variant {prefill_variant} is not one of (0, 1, 3)")
    if len(sizes) != len(expert_ids):
        raise ValueError(f"{len(sizes)} group sizes but {len(expert_ids)} expert ids")
    bm = block_m if (block_m is not None and max((int(m) for m in sizes), default=0) > 1) else None
    return _launch_fwd(_hiplib.FMT_MXFP4, a_cat, blocks, scales, sizes, expert_ids, bm,
                       "gemm_mxfp4_grouped")


def dgrad_mxfp4_grouped(grad_out, blocks, scales, sizes, expert_ids, config=None):
    """``grad_a[t, :] = grad_out[t, :] @ dequant_mxfp4(W[e(t)])`` in one launch.

    Same layouts and ``config`` meaning as ``nf4_grouped.dgrad_4bit_grouped``
    (BLOCK_K must divide 64); the contraction runs in fixed ascending
    64-wide steps of N, so the output bits do not depend on ``config``."""
    blocks = _flat_blocks(blocks)
    E, N, half = blocks.shape
    K = half * 2
    T = grad_out.shape[0]
    assert sum(int(m) for m in sizes) == T, (sum(int(m) for m in sizes), T)
    _require_gpu(grad_out, "dgrad_mxfp4_grouped",
                 "The CPU-checkable equivalent is grad_out @ dequant_mxfp4(...) per group.")
    _bm, _bn, block_k, _w = config or _DGRAD_DEFAULT
    why = None
    if grad_out.dtype != torch.bfloat16:
        why = f"grad_out dtype {grad_out.dtype} is not bfloat16"
    elif 64 % block_k:
        why = f"BLOCK_K {block_k} does not divide 64"
    elif tuple(scales.shape) != (E, N, K // MX_BLOCK) or scales.dtype != torch.uint8:
        why = f"scales {tuple(scales.shape)} {scales.dtype} do not tile K {K} at blocksize {MX_BLOCK}"
    elif grad_out.shape[1] != N:
        why = f"grad_out has {grad_out.shape[1]} columns, blocks have N={N}"
    elif blocks.numel() == 0:
        why = "packed storage is empty (evicted?)"
    if why is not None:
        raise ValueError(f"dgrad_mxfp4_grouped cannot run this problem: {why}.")
    if len(sizes) != len(expert_ids):
        raise ValueError(f"{len(sizes)} group sizes but {len(expert_ids)} expert ids")
    return _launch_dgrad(_hiplib.FMT_MXFP4, grad_out, blocks, scales, sizes, expert_ids,
                         "dgrad_mxfp4_grouped")
