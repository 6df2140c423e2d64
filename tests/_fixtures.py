"""Seeded fixtures and error measures shared by the tests (not a test module)."""
from __future__ import annotations

import numpy as np
import torch


def rand_nf4_stack(E, N, K, seed=0, device="cuda", amax_lo=0.03, amax_hi=0.08):
    """Random packed NF4 bytes and absmax (the kernel's inputs are bytes; a
    quantizer is not needed to exercise the decode)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    B = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8)
    A = torch.rand(E, N, K // 64, generator=g, dtype=torch.float32) * (amax_hi - amax_lo) + amax_lo
    return B.to(device), A.to(device)


def rand_mx_stack(E, N, K, seed=0, device="cuda", e_lo=119, e_hi=125):
    """Random e2m1 bytes and e8m0 scales 2^(e-127), e in [e_lo, e_hi)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    B = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8)
    S = torch.randint(e_lo, e_hi, (E, N, K // 32), generator=g, dtype=torch.uint8)
    return B.to(device), S.to(device)


def rand_acts(T, K, seed=1, device="cuda", std=1.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(T, K, generator=g) * std).to(device=device, dtype=torch.bfloat16)


def spread_ids(E, k):
    return list(range(0, E, max(1, E // k)))[:k]


def dequant(fmt, packed_e, scale_e):
    """fp32 [N, K] decode of one expert, on the tensors' device."""
    if fmt == "nf4":
        from nf4_grouped import dequant_ref
        N, half = packed_e.shape
        return dequant_ref(packed_e, scale_e, N, half * 2)
    from mxfp4_pack_ref import dequant_mxfp4
    N, half = packed_e.shape
    return dequant_mxfp4(packed_e.reshape(N, half // 16, 16), scale_e.reshape(N, half // 16))


def fp64_ref(fmt, a, W, S, sizes, ids):
    outs, row = [], 0
    for m, e in zip(sizes, ids):
        w = dequant(fmt, W[e], S[e]).double()
        outs.append(a[row:row + m].double() @ w.t())
        row += m
    return torch.cat(outs) if outs else torch.zeros(0, W.shape[1], dtype=torch.float64)


def dequant_path(fmt, a, W, S, sizes, ids):
    """The comparator of the tolerance contract: weights materialised in
    bf16, then a bf16 matmul."""
    outs, row = [], 0
    for m, e in zip(sizes, ids):
        wb = dequant(fmt, W[e], S[e]).to(torch.bfloat16)
        outs.append(a[row:row + m] @ wb.t())
        row += m
    return torch.cat(outs)


def rel_err(x, ref) -> float:
    x = x.double()
    ref = ref.double()
    return ((x - ref).norm() / ref.norm().clamp_min(1e-300)).item()


def contract_check(fmt, out, a, W, S, sizes, ids, bound=1e-2, factor=2.0):
    """B-rel (<= factor x the dequant path vs fp64) and B-abs (<= bound)."""
    ref = fp64_ref(fmt, a, W, S, sizes, ids)
    e_f = rel_err(out, ref)
    e_d = rel_err(dequant_path(fmt, a, W, S, sizes, ids), ref)
    assert e_f <= bound, f"B-abs: {e_f:.3e} > {bound}"
    assert e_f <= factor * e_d, f"B-rel: {e_f:.3e} > {factor} x dequant {e_d:.3e}"
    return e_f, e_d


def oracle_fwd(fmt, a, W, S, sizes, ids):
    """The C oracle (locked CPU tree) on the same inputs, fp32 numpy."""
    from oracle import native
    return native.gemv_grouped(a.float().cpu().numpy(), W.cpu().numpy(), S.cpu().numpy(),
                               [int(m) for m in sizes], list(ids), fmt=fmt)


def oracle_dgrad(fmt, g, W, S, sizes, ids):
    from oracle import native
    return native.dgrad_grouped(g.float().cpu().numpy(), W.cpu().numpy(), S.cpu().numpy(),
                                [int(m) for m in sizes], list(ids), fmt=fmt)


def routed_sizes(T_tokens, top_k, E, seed=0, zipf_s=None):
    """Per-expert row counts of top-k routing: uniform distinct experts per
    token, or Zipf(s) popularity over a seeded permutation. Returns
    (sizes, ids) over the active experts in ascending id order."""
    rng = np.random.default_rng(seed)
    counts = np.zeros(E, dtype=np.int64)
    if zipf_s is None:
        for _ in range(T_tokens):
            counts[rng.choice(E, size=top_k, replace=False)] += 1
    else:
        p = 1.0 / np.arange(1, E + 1) ** zipf_s
        p = p[rng.permutation(E)]
        p /= p.sum()
        for _ in range(T_tokens):
            counts[rng.choice(E, size=top_k, replace=False, p=p)] += 1
    ids = [int(e) for e in np.nonzero(counts)[0]]
    return [int(counts[e]) for e in ids], ids
