"""fp16 and fp32 activations on the forward ops.

The reference's kernels load activations of any float dtype and widen them in
registers (kernel/nf4_grouped.py:456-458, 511; kernel/mxfp4_grouped.py:94;
docs/KERNEL_CONTRACT.md:25 lists A in {fp16, bf16, fp32}). Here they are
rounded once to bf16, nearest-even, by the library's widening kernel, and
then take the bf16 kernels. Bars:
  * the widening is bit-exact against torch's ``.to(bfloat16)`` (subnormals,
    infinities, ties and the overflow edge included; NaN stays NaN);
  * the forward of fp16/fp32 input equals the forward of ``a.to(bf16)`` bit
    for bit, on the decode and the tiled kernels;
  * against fp64 on the ORIGINAL input: B-abs <= 1e-2 and B-rel <= 2x the
    bf16 dequant-then-matmul path; against the C oracle (fp32 activations,
    the reference's CPU tier) within 1e-2 relative.
"""
import struct

import pytest
import torch

from _fixtures import dequant, fp64_ref, oracle_fwd, rand_mx_stack, rand_nf4_stack, rel_err

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.float32]


def _ops():
    from mxfp4_grouped import gemm_mxfp4_grouped
    from nf4_grouped import gemm_4bit_grouped
    return {"nf4": gemm_4bit_grouped, "mxfp4": gemm_mxfp4_grouped}


def _stack(fmt, E, N, K, seed=0):
    return rand_nf4_stack(E, N, K, seed) if fmt == "nf4" else rand_mx_stack(E, N, K, seed)


def _widen(src):
    import _hiplib
    from nf4_grouped import _WIDEN_DTYPES
    T, K = src.shape
    dst = torch.empty(T, K, dtype=torch.bfloat16, device=src.device)
    rc = _hiplib.load().gnf4_hip_activations_to_bf16(
        src.data_ptr(), _WIDEN_DTYPES[src.dtype], T, K, src.stride(0), dst.data_ptr(),
        dst.stride(0), torch.cuda.current_stream().cuda_stream)
    _hiplib.check(rc, "widen")
    return dst


def _edge_values(dtype):
    fi = torch.finfo(dtype)
    vals = [0.0, -0.0, 1.0, -1.0, fi.tiny, -fi.tiny, fi.max, -fi.max, float("inf"),
            float("-inf"), fi.tiny / 4, fi.eps, 1.0 + fi.eps]
    if dtype == torch.float32:
        # exact ties between two bf16 values (odd and even lower neighbours),
        # one ulp either side of a tie, and the largest value that still
        # rounds to a finite bf16
        for bits in (0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0x7F7F7FFF, 0x7F7F8000,
                     0x00008000, 0x00018000, 0x80008000):
            vals.append(struct.unpack("<f", struct.pack("<I", bits))[0])
    return torch.tensor(vals, dtype=dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_widening_is_bitwise_torch_rounding(dtype):
    g = torch.Generator().manual_seed(5)
    body = (torch.randn(37 * 256, generator=g) * torch.logspace(-30, 30, 37 * 256) ** 0.3)
    if dtype == torch.float16:
        body = body.clamp(-6e4, 6e4)
    vals = torch.cat([_edge_values(dtype), body.to(dtype)])
    pad = (-vals.numel()) % 256
    vals = torch.cat([vals, torch.zeros(pad, dtype=dtype)]).reshape(-1, 256).cuda()
    got = _widen(vals)
    want = vals.to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("dtype", DTYPES)
def test_widening_nan_and_strided_rows(dtype):
    x = torch.randn(6, 72, device="cuda").to(dtype)
    x[2, 5] = float("nan")
    big = torch.zeros(6, 80, device="cuda", dtype=dtype)
    big[:, :72] = x
    got = _widen(big[:, :72])              # row stride 80, 72 columns
    assert torch.isnan(got[2, 5]).item()
    x[2, 5] = 0
    got[2, 5] = 0
    assert torch.equal(got.view(torch.int16), x.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("sizes", [[1] * 6, [3, 16, 1, 7, 2, 5], [40, 1, 130, 3, 66, 9]])
def test_forward_equals_the_bf16_forward_bitwise(fmt, dtype, sizes):
    N, K, E = 256, 512, 8
    W, S = _stack(fmt, E, N, K, seed=21)
    ids = [5, 0, 7, 2, 3, 6]
    g = torch.Generator().manual_seed(22)
    a = (torch.randn(sum(sizes), K, generator=g) * 3).to(dtype).cuda()
    op = _ops()[fmt]
    out = op(a, W, S, sizes, ids)
    ref = op(a.to(torch.bfloat16), W, S, sizes, ids)
    assert out.dtype == torch.bfloat16
    assert torch.equal(out, ref)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 128])
def test_contract_against_fp64_of_the_original_input(fmt, dtype, m):
    N, K, E = 768, 2048, 8
    W, S = _stack(fmt, E, N, K, seed=31)
    ids = [1, 4, 6]
    sizes = [m] * len(ids)
    g = torch.Generator().manual_seed(32)
    a = torch.randn(sum(sizes), K, generator=g).to(dtype).cuda()
    out = _ops()[fmt](a, W, S, sizes, ids)
    ref = fp64_ref(fmt, a, W, S, sizes, ids)
    ab = a.to(torch.bfloat16)
    outs, row = [], 0
    for mm, e in zip(sizes, ids):
        outs.append(ab[row:row + mm] @ dequant(fmt, W[e], S[e]).to(torch.bfloat16).t())
        row += mm
    e_f, e_d = rel_err(out, ref), rel_err(torch.cat(outs), ref)
    assert e_f <= 1e-2, f"B-abs: {e_f:.3e}"
    assert e_f <= 2.0 * e_d, f"B-rel: {e_f:.3e} > 2 x dequant {e_d:.3e}"
    orc = torch.from_numpy(oracle_fwd(fmt, a, W, S, sizes, ids))
    assert rel_err(out.float().cpu(), orc) < 1e-2


def test_planned_launch_takes_fp16():
    from nf4_grouped import GroupPlan, launch_planned
    import _hiplib
    N, K, E = 256, 256, 4
    W, S = rand_nf4_stack(E, N, K, seed=41)
    sizes, ids = [2, 5, 1], [3, 0, 2]
    a = torch.randn(sum(sizes), K, device="cuda").half()
    plan = GroupPlan(sizes, ids, "cuda")
    out = launch_planned(_hiplib.FMT_NF4, a, W, S, plan)
    assert torch.equal(out, launch_planned(_hiplib.FMT_NF4, a.to(torch.bfloat16), W, S, plan))


def test_other_activation_dtypes_are_refused():
    from nf4_grouped import gemm_4bit_grouped
    W, S = rand_nf4_stack(2, 64, 64, seed=1)
    with pytest.raises(TypeError):
        gemm_4bit_grouped(torch.zeros(2, 64, dtype=torch.float64, device="cuda"), W, S,
                          [1, 1], [0, 1])
