"""LoRA delta of the QLoRA training path, checked on the CPU (pure torch).

Mirrors the reference's kernel/test_nf4_qlora_grad.py:53-105, :228-284
(explicit per-expert math, the alpha/r scaling, zero-B, batched == loop,
pathological skew falls back to the loop, no rows -> None)."""
import pytest
import torch

import nf4_qlora
from nf4_qlora import _lora_delta_grouped_loop, lora_delta_grouped


def _case(sizes, E=6, K=40, N=24, r=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(sum(sizes), K, generator=g)
    A = torch.randn(E, r, K, generator=g)
    B = torch.randn(E, N, r, generator=g)
    return a, A, B


def _explicit(a, A, B, sizes, ids, scaling):
    out, row = torch.zeros(a.shape[0], B.shape[1]), 0
    for m, e in zip(sizes, ids):
        for t in range(row, row + m):
            out[t] = scaling * (B[e] @ (A[e] @ a[t]))
        row += m
    return out


@pytest.mark.parametrize("sizes,ids", [([3, 1, 4], [2, 0, 5]), ([5, 0, 2, 2], [1, 3, 4, 0]),
                                       ([1], [3])])
def test_delta_matches_explicit_per_expert_math(sizes, ids):
    a, A, B = _case(sizes)
    d = lora_delta_grouped(a, A, B, sizes, ids, scaling=0.5)
    torch.testing.assert_close(d, _explicit(a, A, B, sizes, ids, 0.5), rtol=1e-5, atol=1e-5)


def test_scaling_is_alpha_over_r():
    sizes, ids = [2, 3], [1, 4]
    a, A, B = _case(sizes)
    one = lora_delta_grouped(a, A, B, sizes, ids, scaling=1.0)
    two = lora_delta_grouped(a, A, B, sizes, ids, scaling=16 / 8)
    torch.testing.assert_close(two, 2.0 * one)


def test_zero_B_delta_is_exactly_zero():
    sizes, ids = [2, 3], [1, 4]
    a, A, B = _case(sizes)
    assert not lora_delta_grouped(a, A, torch.zeros_like(B), sizes, ids).any()


@pytest.mark.parametrize("sizes,ids", [([4, 4, 4], [0, 1, 2]), ([3, 5, 1, 2], [5, 1, 0, 3]),
                                       ([2, 0, 7], [4, 2, 1])])
def test_batched_delta_matches_the_loop(sizes, ids):
    a, A, B = _case(sizes, seed=3)
    torch.testing.assert_close(lora_delta_grouped(a, A, B, sizes, ids, 0.25),
                               _lora_delta_grouped_loop(a, A, B, sizes, ids, 0.25),
                               rtol=1e-5, atol=1e-5)


def test_pathological_skew_falls_back_to_the_loop(monkeypatch):
    sizes, ids = [40, 1, 1, 1, 1, 1], [0, 1, 2, 3, 4, 5]   # 6 x 40 padded rows for 45 real
    a, A, B = _case(sizes)
    calls = []
    orig = nf4_qlora._lora_delta_grouped_loop

    def spy(*args, **kw):
        calls.append(1)
        return orig(*args, **kw)

    monkeypatch.setattr(nf4_qlora, "_lora_delta_grouped_loop", spy)
    d = nf4_qlora.lora_delta_grouped(a, A, B, sizes, ids)
    assert calls == [1]
    torch.testing.assert_close(d, _explicit(a, A, B, sizes, ids, 1.0), rtol=1e-5, atol=1e-5)


def test_no_rows_returns_none():
    a, A, B = _case([0, 0])
    assert lora_delta_grouped(a, A, B, [0, 0], [1, 2]) is None
    assert _lora_delta_grouped_loop(a, A, B, [0, 0], [1, 2]) is None


def test_delta_is_differentiable_in_A_and_B():
    sizes, ids = [2, 3], [1, 4]
    a, A, B = _case(sizes)
    A.requires_grad_(True)
    B.requires_grad_(True)
    lora_delta_grouped(a, A, B, sizes, ids).square().sum().backward()
    assert A.grad is not None and A.grad[1].abs().sum() > 0 and A.grad[0].abs().sum() == 0
    assert B.grad is not None and B.grad[4].abs().sum() > 0
