"""QLoRA training path on the GPU: forward bits, input gradient through the
dgrad kernel and through the exact per-expert loop, LoRA parameter gradients,
offload-style weights_fn (reference kernel/test_nf4_qlora_grad.py:108-384)."""
import pytest
import torch

from _fixtures import dequant, rand_acts, rand_mx_stack, rand_nf4_stack, rel_err

pytestmark = pytest.mark.gpu


def _stack(fmt, E, N, K, seed=0):
    return rand_nf4_stack(E, N, K, seed) if fmt == "nf4" else rand_mx_stack(E, N, K, seed)


def _train(fmt):
    import nf4_qlora
    return nf4_qlora.gemm_4bit_grouped_train if fmt == "nf4" else nf4_qlora.gemm_mxfp4_grouped_train


def _grad_fp64(fmt, go, W, S, sizes, ids):
    outs, row = [], 0
    for m, e in zip(sizes, ids):
        outs.append(go[row:row + m].double() @ dequant(fmt, W[e], S[e]).double())
        row += m
    return torch.cat(outs)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("dgrad_kernel", [True, False])
def test_input_gradient_matches_fp64(fmt, dgrad_kernel):
    from mxfp4_grouped import gemm_mxfp4_grouped
    from nf4_grouped import gemm_4bit_grouped
    W, S = _stack(fmt, 6, 256, 512)
    sizes, ids = [40, 3, 130, 0, 17], [5, 0, 2, 1, 3]
    a = rand_acts(sum(sizes), 512).requires_grad_(True)
    out = _train(fmt)(a, W, S, sizes, ids, dgrad_kernel=dgrad_kernel)
    plain = (gemm_4bit_grouped if fmt == "nf4" else gemm_mxfp4_grouped)(a.detach(), W, S, sizes, ids)
    assert torch.equal(out.detach(), plain)
    go = rand_acts(sum(sizes), 256, seed=9, std=1e-2)
    out.backward(go)
    ref = _grad_fp64(fmt, go, W, S, sizes, ids)
    assert rel_err(a.grad, ref) <= 1e-2


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_kernel_and_exact_loop_agree_within_the_bf16_budget(fmt):
    W, S = _stack(fmt, 4, 512, 1024, seed=4)
    sizes, ids = [64, 200, 5], [3, 1, 0]
    grads = []
    for dk in (True, False):
        a = rand_acts(sum(sizes), 1024, seed=5).requires_grad_(True)
        _train(fmt)(a, W, S, sizes, ids, dgrad_kernel=dk).backward(
            rand_acts(sum(sizes), 512, seed=6, std=1e-2))
        grads.append(a.grad.float())
    assert rel_err(grads[0], grads[1]) <= 1e-2


def test_weights_fn_is_read_at_backward_time():
    import nf4_qlora
    W, S = _stack("nf4", 4, 256, 512, seed=2)
    sizes, ids = [9, 20], [2, 0]
    a1 = rand_acts(29, 512).requires_grad_(True)
    a2 = rand_acts(29, 512).requires_grad_(True)
    go = rand_acts(29, 256, seed=3, std=1e-2)
    fetched = []

    def weights_fn():
        fetched.append(1)
        return W, S

    nf4_qlora.gemm_4bit_grouped_train(a1, W, S, sizes, ids).backward(go)
    out = nf4_qlora.gemm_4bit_grouped_train(a2, W, S, sizes, ids, weights_fn=weights_fn)
    assert fetched == []
    out.backward(go)
    assert fetched == [1]
    assert torch.equal(a1.grad, a2.grad)


def test_lora_parameters_receive_gradients_through_the_fused_path():
    import nf4_qlora
    E, N, K, r = 4, 256, 512, 8
    W, S = _stack("nf4", E, N, K, seed=7)
    sizes, ids = [12, 0, 30], [1, 3, 2]
    a = rand_acts(sum(sizes), K, seed=8)
    g = torch.Generator(device="cpu").manual_seed(1)
    lA = (torch.randn(E, r, K, generator=g) * 0.02).cuda().requires_grad_(True)
    lB = (torch.randn(E, N, r, generator=g) * 0.02).cuda().requires_grad_(True)
    x = a.clone().requires_grad_(True)
    out = nf4_qlora.fused_grouped_lora(x, W, S, sizes, ids, lora_A=lA, lora_B=lB, scaling=2.0)
    go = rand_acts(sum(sizes), N, seed=10, std=1e-2)
    out.backward(go)
    # fp64 reference of the same composition
    xr = a.double().requires_grad_(True)
    Ar, Br = lA.detach().double().requires_grad_(True), lB.detach().double().requires_grad_(True)
    ref, row = [], 0
    for m, e in zip(sizes, ids):
        xs = xr[row:row + m]
        w = dequant("nf4", W[e], S[e]).double()
        ref.append(xs @ w.t() + 2.0 * (xs @ Ar[e].t()) @ Br[e].t())
        row += m
    ref = torch.cat(ref)
    ref.backward(go.double())
    assert rel_err(out, ref.detach()) <= 1e-2
    assert rel_err(x.grad, xr.grad) <= 1e-2
    assert rel_err(lA.grad, Ar.grad) <= 1e-2 and rel_err(lB.grad, Br.grad) <= 1e-2
    assert not lA.grad[0].any() and lA.grad[1].any()   # only the routed experts
