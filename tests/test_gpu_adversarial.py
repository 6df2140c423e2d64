"""Adversarial absmax / scale values on every NF4 kernel family.

Reference: kernel/test_nf4_grouped.py:142-161 (tiny 1e-30, huge 1e30, mixed
alternating rows, denormal-adjacent 1e-38; relative error vs fp64 <= 1e-2 and
a finite output) and kernel/test_interp_contract.py:97-106 (one block with a
1e3 outlier). The contract (docs/TOLERANCE_CONTRACT.md, property test 2)
asks that the codebook x absmax multiply neither flush nor overflow
differently from the dequant path.

Row counts pick the kernel: 1 row per group runs the fp32 FMA decode path,
5 and 12 rows the split-codebook MFMA decode (one and two row sets), 40 rows
the 128-row tiles, 300 rows the 256-row tiles; dgrad runs its 256-row tiles
and, with K = 96, its 128-row fallback.
"""
import pytest
import torch

from _fixtures import dequant, fp64_ref, rel_err

pytestmark = pytest.mark.gpu

KINDS = ["tiny", "huge", "mixed", "denormal_adj"]


def _absmax(kind, E, N, K):
    val = {"tiny": 1e-30, "huge": 1e30, "denormal_adj": 1e-38}.get(kind)
    A = torch.full((E, N, K // 64), val or 1.0, dtype=torch.float32, device="cuda")
    if kind == "mixed":
        A[:, ::2, :] = 1e30
        A[:, 1::2, :] = 1e-30
    return A


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows", [1, 5, 12, 40, 300])
def test_forward_absmax_extremes(kind, rows):
    from nf4_grouped import gemm_4bit_grouped
    N, K, E = 64, 128, 2
    g = torch.Generator().manual_seed(3)
    B = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8).cuda()
    A = _absmax(kind, E, N, K)
    a = (torch.randn(2 * rows, K, generator=g) * 0.5).to("cuda", torch.bfloat16)
    out = gemm_4bit_grouped(a, B, A, [rows, rows], [0, 1])
    assert torch.isfinite(out.float()).all()
    e = rel_err(out, fp64_ref("nf4", a, B, A, [rows, rows], [0, 1]))
    assert e <= 1e-2, f"{kind} rows={rows}: rel err {e:.2e}"


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("K", [128, 96 * 2])
def test_dgrad_absmax_extremes(kind, K):
    """dgrad: dX = dY . W with the same absmax extremes; K = 128 runs the
    four-wave transposed-read tiles, K = 192 with N = 96 (not a multiple of
    64) the fallback tile kernel."""
    from nf4_grouped import dgrad_4bit_grouped, dequant_ref
    N = 64 if K == 128 else 96
    E, rows = 2, 150
    g = torch.Generator().manual_seed(4)
    B = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8).cuda()
    A = _absmax(kind, E, N, K)
    go = (torch.randn(2 * rows, N, generator=g) * 0.5).to("cuda", torch.bfloat16)
    out = dgrad_4bit_grouped(go, B, A, [rows, rows], [0, 1])
    assert torch.isfinite(out.float()).all()
    ref = torch.cat([go[e * rows:(e + 1) * rows].double() @ dequant_ref(B[e], A[e], N, K).double()
                     for e in range(E)])
    e = rel_err(out, ref)
    assert e <= 1e-2, f"{kind} K={K}: rel err {e:.2e}"


@pytest.mark.parametrize("rows", [1, 5, 40, 300])
def test_single_block_outlier(rows):
    """One 64-element block per row carries a 1e3 x larger absmax than the
    rest (reference kernel/test_interp_contract.py:97-106): per-block
    scaling must keep the small blocks' contribution. Max-abs error relative
    to the largest output, as the reference measures it."""
    from nf4_grouped import gemm_4bit_grouped
    N, K = 64, 128
    g = torch.Generator().manual_seed(7)
    B = torch.randint(0, 256, (2, N, K // 2), generator=g, dtype=torch.uint8).cuda()
    A = (torch.rand(2, N, K // 64, generator=g) * 0.05 + 0.01).cuda()
    A[0, :, 0] *= 1e3
    a = torch.randn(rows, K, generator=g).to("cuda", torch.bfloat16)
    out = gemm_4bit_grouped(a, B, A, [rows], [0])
    ref = a.double() @ dequant("nf4", B[0], A[0]).double().t()
    err = (out.double() - ref).abs().max() / ref.abs().max().clamp_min(1e-4)
    assert err < 1e-2
