"""Differentiable grouped 4-bit expert projection for QLoRA training.

The frozen base weight stays packed. Forward runs the grouped forward kernel;
backward needs only the input gradient ``grad_out @ W`` (the base weight is
not trained), which the grouped dgrad kernel computes from the same packed
bytes in one launch. No decoded weight is kept between forward and backward.

LoRA composes pre-activation: ``fused_grouped_lora`` returns
``W x + scaling * B (A x)`` per group, so a caller applies SwiGLU after it.

Interface and semantics follow the reference's kernel/nf4_qlora.py:32-305
(``FusedGroupedNf4``, ``gemm_4bit_grouped_train``, ``lora_delta_grouped``,
``_lora_delta_grouped_loop``, ``fused_grouped_lora``, ``_PAD_WASTE_LIMIT``).
"""
from __future__ import annotations

import torch

import mxfp4_grouped
import nf4_grouped

# Padded-bmm cutoff for lora_delta_grouped: above this many padded rows per
# real row the per-expert loop is used instead (reference nf4_qlora.py:26-30).
_PAD_WASTE_LIMIT = 4.0


def _host_ints(x):
    """A host list of ints from a list, tuple or tensor (one transfer)."""
    if isinstance(x, (list, tuple)):
        return [int(v) for v in x]
    return [int(v) for v in x.tolist()]


def _exact_dgrad_loop(grad_out, packed, scales, sizes, expert_ids, decode):
    """grad_a = grad_out @ decode(W[e]) one group at a time, each decoded
    expert dropped before the next (the reference's exact backward,
    nf4_qlora.py:137-166). Runs where grad_out lives; the weights of one
    expert are moved there if they are stored elsewhere."""
    _E, N, half = packed.shape
    K = half * 2
    grad_a = torch.empty(grad_out.shape[0], K, dtype=grad_out.dtype, device=grad_out.device)
    sizes_h, eids_h = _host_ints(sizes), _host_ints(expert_ids)
    row = 0
    for g, e in enumerate(eids_h):
        m = sizes_h[g]
        if m == 0:
            continue
        pe = packed[e].to(grad_out.device, non_blocking=True)
        se = scales[e].to(grad_out.device, non_blocking=True)
        w = decode(pe, se, N, K).to(grad_out.dtype)
        grad_a[row:row + m] = grad_out[row:row + m] @ w
        del pe, se, w
        row += m
    return grad_a


class FusedGroupedNf4(torch.autograd.Function):
    """Grouped NF4 forward through the kernel; input gradient through the
    grouped dgrad kernel (or, with ``dgrad_kernel=False``, through the exact
    per-expert decode). ``packed`` / ``absmax`` are constants: they are kept
    on ctx (or re-fetched from ``weights_fn`` at backward time, so offloaded
    storage is not pinned by a reference here), never saved for gradient."""

    @staticmethod
    def forward(ctx, a_cat, packed, absmax, sizes, expert_ids, weights_fn=None,
                dgrad_kernel=True):
        out = nf4_grouped.gemm_4bit_grouped(a_cat, packed, absmax, sizes, expert_ids)
        ctx.weights_fn = weights_fn
        ctx.packed, ctx.absmax = (packed, absmax) if weights_fn is None else (None, None)
        ctx.sizes, ctx.expert_ids = sizes, expert_ids   # as given: no device reads here
        ctx.dgrad_kernel = dgrad_kernel
        return out

    @staticmethod
    def backward(ctx, grad_out):
        if not ctx.needs_input_grad[0]:
            return (None,) * 7
        packed, absmax = ((ctx.packed, ctx.absmax) if ctx.weights_fn is None
                          else ctx.weights_fn())
        grad_out = grad_out.contiguous()
        if (ctx.dgrad_kernel and packed.device == grad_out.device
                and nf4_grouped.dgrad_eligible(grad_out, packed, absmax) is None):
            grad_a = nf4_grouped.dgrad_4bit_grouped(grad_out, packed, absmax,
                                                    ctx.sizes, ctx.expert_ids)
        else:
            grad_a = _exact_dgrad_loop(grad_out, packed, absmax, ctx.sizes, ctx.expert_ids,
                                       nf4_grouped.dequant_ref)
        return (grad_a,) + (None,) * 6


def gemm_4bit_grouped_train(a_cat, packed, absmax, sizes, expert_ids, weights_fn=None,
                            dgrad_kernel=True):
    """``gemm_4bit_grouped`` with a gradient for ``a_cat`` (reference
    nf4_qlora.py:168-178). ``weights_fn``: zero-argument callable returning
    ``(packed, absmax)`` at backward time, for offload-staged storage."""
    return FusedGroupedNf4.apply(a_cat, packed, absmax, sizes, expert_ids, weights_fn,
                                 dgrad_kernel)


class FusedGroupedMxfp4(torch.autograd.Function):
    """The MXFP4 counterpart: forward and input gradient both through the
    kernels (the reference's GPU backward is a per-expert decode loop,
    kernel/mxfp4_qlora.py:106-122; ``dgrad_kernel=False`` keeps that)."""

    @staticmethod
    def forward(ctx, a_cat, blocks, scales, sizes, expert_ids, weights_fn=None,
                dgrad_kernel=True):
        out = mxfp4_grouped.gemm_mxfp4_grouped(a_cat, blocks, scales, sizes, expert_ids)
        ctx.weights_fn = weights_fn
        ctx.blocks, ctx.scales = (blocks, scales) if weights_fn is None else (None, None)
        ctx.sizes, ctx.expert_ids = sizes, expert_ids
        ctx.dgrad_kernel = dgrad_kernel
        return out

    @staticmethod
    def backward(ctx, grad_out):
        if not ctx.needs_input_grad[0]:
            return (None,) * 7
        blocks, scales = ((ctx.blocks, ctx.scales) if ctx.weights_fn is None
                          else ctx.weights_fn())
        grad_out = grad_out.contiguous()
        flat = mxfp4_grouped._flat_blocks(blocks)
        if ctx.dgrad_kernel and flat.device == grad_out.device:
            grad_a = mxfp4_grouped.dgrad_mxfp4_grouped(grad_out, flat, scales, ctx.sizes,
                                                       ctx.expert_ids)
        else:
            from mxfp4_pack_ref import dequant_mxfp4

            def decode(pe, se, n, k):
                return dequant_mxfp4(pe.reshape(n, k // 32, 16), se.reshape(n, k // 32))

            grad_a = _exact_dgrad_loop(grad_out, flat, scales, ctx.sizes, ctx.expert_ids,
                                       decode)
        return (grad_a,) + (None,) * 6


def gemm_mxfp4_grouped_train(a_cat, blocks, scales, sizes, expert_ids, weights_fn=None,
                             dgrad_kernel=True):
    """``gemm_mxfp4_grouped`` with a gradient for ``a_cat``."""
    return FusedGroupedMxfp4.apply(a_cat, blocks, scales, sizes, expert_ids, weights_fn,
                                   dgrad_kernel)


def lora_delta_grouped(a_cat, lora_A, lora_B, sizes, expert_ids, scaling=1.0):
    """Per-group low-rank delta ``scaling * (x @ A[e].T) @ B[e].T`` over a
    group-sorted block (reference nf4_qlora.py:181-254). ``lora_A`` is
    ``[E, r, K]``, ``lora_B`` ``[E, N, r]``; returns ``[T, N]`` or ``None``
    when no group has rows. Groups are padded to the widest and run as two
    batched matmuls; when padding would exceed ``_PAD_WASTE_LIMIT`` times the
    real rows, the per-group loop runs instead. ``expert_ids`` on the device
    is never read on the host."""
    nz = [g for g in range(len(sizes)) if int(sizes[g]) > 0]
    if not nz:
        return None
    rows = [int(sizes[g]) for g in nz]
    total, widest = sum(rows), max(rows)
    if len(rows) * widest > _PAD_WASTE_LIMIT * total:
        return _lora_delta_grouped_loop(a_cat, lora_A, lora_B, sizes, expert_ids, scaling)
    dev = a_cat.device
    if torch.is_tensor(expert_ids) and expert_ids.device.type != "cpu":
        sz_d, nz_d = nf4_grouped.to_device_i32((rows, nz), dev)
        eid = expert_ids.to(dev)[nz_d.to(torch.int64)].to(torch.int64)
    else:
        ids = _host_ints(expert_ids)
        sz_d, eid_d = nf4_grouped.to_device_i32((rows, [ids[g] for g in nz]), dev)
        eid = eid_d.to(torch.int64)
    sz = sz_d.to(torch.int64)
    # row -> (group, position in group), built on the device; output_size
    # keeps repeat_interleave from reading sz on the host
    grp = torch.repeat_interleave(torch.arange(len(rows), device=dev), sz, output_size=total)
    start = torch.cumsum(sz, 0) - sz
    pos = torch.arange(total, device=dev) - start[grp]
    A, B = lora_A[eid], lora_B[eid]                        # [G, r, K], [G, N, r]
    x = a_cat.new_zeros(len(rows), widest, a_cat.shape[1], dtype=A.dtype)
    x[grp, pos] = a_cat[:total].to(A.dtype)
    d = scaling * torch.bmm(torch.bmm(x, A.transpose(1, 2)), B.transpose(1, 2))
    out = torch.zeros(a_cat.shape[0], B.shape[1], dtype=d.dtype, device=dev)
    out[:total] = d[grp, pos]
    return out


def _lora_delta_grouped_loop(a_cat, lora_A, lora_B, sizes, expert_ids, scaling=1.0):
    """Per-group reference for ``lora_delta_grouped`` (reference
    nf4_qlora.py:257-283); the fallback for heavily skewed groups."""
    out = None
    row = 0
    for g, e in enumerate(_host_ints(expert_ids)):
        m = int(sizes[g])
        if m == 0:
            continue
        A, B = lora_A[e], lora_B[e]
        d = scaling * ((a_cat[row:row + m].to(A.dtype) @ A.T) @ B.T)
        if out is None:
            out = torch.zeros(a_cat.shape[0], B.shape[0], dtype=d.dtype, device=a_cat.device)
        out[row:row + m] = d
        row += m
    return out


def fused_grouped_lora(a_cat, packed, absmax, sizes, expert_ids, lora_A=None, lora_B=None,
                       weights_fn=None, scaling=1.0, dgrad_kernel=True):
    """Frozen NF4 projection plus the trainable delta, pre-activation
    (reference nf4_qlora.py:286-305): differentiable in ``a_cat``, ``lora_A``
    and ``lora_B``."""
    out = gemm_4bit_grouped_train(a_cat, packed, absmax, sizes, expert_ids,
                                  weights_fn=weights_fn, dgrad_kernel=dgrad_kernel)
    if lora_A is None or lora_B is None:
        return out
    delta = lora_delta_grouped(a_cat, lora_A, lora_B, sizes, expert_ids, scaling)
    return out if delta is None else out + delta.to(out.dtype)
