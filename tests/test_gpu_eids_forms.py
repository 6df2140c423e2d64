"""Every `expert_ids` form gives the same bits, on every entry point.

Restates kernel/test_eids_forms.py:66-92: a Python list, a host int32
tensor and a device int32 tensor of the same ids give bitwise-equal results
for the forward, the dgrad, the LoRA delta and the fused training backward
(jagged sizes with an empty group). Weights are quantized by the fixture
packer (the reference quantizes with bitsandbytes, absent here; the property
is about the id carrier, not the weights). Both formats; the fused FFN's
own form test is in test_gpu_ffn.py.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

E, N, K, RANK = 8, 128, 128, 4
SIZES = [3, 1, 0, 5, 2]              # jagged, with an empty group
EIDS = [0, 3, 7, 5, 2]


@pytest.fixture(scope="module")
def fx():
    from mxfp4_pack_ref import quantize_pack_mxfp4
    from nf4_pack_ref import quantize_pack_nf4
    g = torch.Generator(device="cpu").manual_seed(7)
    w = torch.randn(E, N, K, generator=g) * 0.02
    nb = torch.empty(E, N, K // 2, dtype=torch.uint8, device="cuda")
    na = torch.empty(E, N, K // 64, dtype=torch.float32, device="cuda")
    mb = torch.empty(E, N, K // 2, dtype=torch.uint8, device="cuda")
    ms = torch.empty(E, N, K // 32, dtype=torch.uint8, device="cuda")
    for e in range(E):
        nb[e], na[e] = quantize_pack_nf4(w[e].cuda())
        b, s = quantize_pack_mxfp4(w[e].cuda())
        mb[e], ms[e] = b.reshape(N, K // 2), s
    a_cat = (torch.randn(sum(SIZES), K, generator=g) * 0.5).to("cuda", torch.bfloat16)
    go = (torch.randn(sum(SIZES), N, generator=g) * 0.1).to("cuda", torch.bfloat16)
    lA = (torch.randn(E, RANK, K, generator=g) * 0.01).to("cuda", torch.bfloat16)
    lB = (torch.randn(E, N, RANK, generator=g) * 0.01).to("cuda", torch.bfloat16)
    return {"nf4": (nb, na), "mxfp4": (mb, ms)}, a_cat, go, lA, lB


def forms():
    return {
        "list": EIDS,
        "cpu_tensor": torch.tensor(EIDS, dtype=torch.int32),
        "cuda_tensor": torch.tensor(EIDS, dtype=torch.int32, device="cuda"),
    }


def _assert_all_equal(outs: dict):
    ref_name, ref = next(iter(outs.items()))
    for name, o in outs.items():
        assert torch.equal(o, ref), (
            f"expert_ids form {name!r} diverged from {ref_name!r}: "
            f"max|d|={(o.float() - ref.float()).abs().max().item():.3e}")


def _fwd(fmt):
    if fmt == "nf4":
        from nf4_grouped import gemm_4bit_grouped
        return gemm_4bit_grouped
    from mxfp4_grouped import gemm_mxfp4_grouped
    return gemm_mxfp4_grouped


def _dgrad(fmt):
    if fmt == "nf4":
        from nf4_grouped import dgrad_4bit_grouped
        return dgrad_4bit_grouped
    from mxfp4_grouped import dgrad_mxfp4_grouped
    return dgrad_mxfp4_grouped


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_forward_identical_across_eids_forms(fx, fmt):
    W, a_cat = fx[0][fmt], fx[1]
    _assert_all_equal({n: _fwd(fmt)(a_cat, *W, SIZES, e) for n, e in forms().items()})


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_identical_across_eids_forms(fx, fmt):
    W, go = fx[0][fmt], fx[2]
    _assert_all_equal({n: _dgrad(fmt)(go, *W, SIZES, e) for n, e in forms().items()})


def test_lora_delta_identical_across_eids_forms(fx):
    from nf4_qlora import lora_delta_grouped
    _w, a_cat, _go, lA, lB = fx
    _assert_all_equal({n: lora_delta_grouped(a_cat, lA, lB, SIZES, e, 2.0)
                       for n, e in forms().items()})


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_fused_train_backward_identical_across_eids_forms(fx, fmt):
    from nf4_qlora import gemm_4bit_grouped_train, gemm_mxfp4_grouped_train
    train = gemm_4bit_grouped_train if fmt == "nf4" else gemm_mxfp4_grouped_train
    W, a_cat = fx[0][fmt], fx[1]
    grads = {}
    for n, e in forms().items():
        x = a_cat.detach().clone().requires_grad_(True)
        out = train(x, *W, SIZES, e, dgrad_kernel=True)
        out.float().pow(2).mean().backward()
        grads[n] = x.grad.detach()
    _assert_all_equal(grads)


def test_fused_lora_backward_identical_across_eids_forms(fx):
    from nf4_qlora import fused_grouped_lora
    (W, _m), a_cat, _go, lA, lB = fx[0]["nf4"], fx[1], fx[2], fx[3], fx[4]
    grads = {}
    for n, e in forms().items():
        x = a_cat.detach().clone().requires_grad_(True)
        la = lA.detach().clone().requires_grad_(True)
        lb = lB.detach().clone().requires_grad_(True)
        out = fused_grouped_lora(x, W, _m, SIZES, e, la, lb, scaling=2.0)
        out.float().pow(2).mean().backward()
        grads[n] = torch.cat([x.grad.flatten(), la.grad.flatten(), lb.grad.flatten()])
    _assert_all_equal(grads)
