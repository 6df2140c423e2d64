"""GPU parity of the dgrad ops (grad_a = grad_out . dequant(W)).

Bars (reference kernel/test_nf4_grouped.py:326-400): agreement with the
per-expert decode oracle within the bf16 budget; output bitwise independent
of the tile config; eligibility decidable before launch. Added here: one-hot
exactness (a one-hot grad row selects one decoded weight row), the C
oracle's ascending-n chain, and the same bars for MXFP4.
"""
import pytest
import torch

from _fixtures import (dequant, oracle_dgrad, rand_acts, rand_mx_stack, rand_nf4_stack,
                       rel_err)

pytestmark = pytest.mark.gpu


def _ops():
    from mxfp4_grouped import dgrad_mxfp4_grouped
    from nf4_grouped import dgrad_4bit_grouped
    return {"nf4": dgrad_4bit_grouped, "mxfp4": dgrad_mxfp4_grouped}


def _stack(fmt, E, N, K, seed=0):
    return rand_nf4_stack(E, N, K, seed) if fmt == "nf4" else rand_mx_stack(E, N, K, seed)


def _oracle_bf16_path(fmt, go, W, S, sizes, ids):
    """What the kernel replaces: decode each expert to bf16, dense matmul."""
    outs, row = [], 0
    for m, e in zip(sizes, ids):
        w = dequant(fmt, W[e], S[e]).to(go.dtype)
        outs.append(go[row:row + m] @ w)
        row += m
    return torch.cat(outs)


def _fp64(fmt, go, W, S, sizes, ids):
    outs, row = [], 0
    for m, e in zip(sizes, ids):
        w = dequant(fmt, W[e], S[e]).double()
        outs.append(go[row:row + m].double() @ w)
        row += m
    return torch.cat(outs)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("rows", [(3, 3, 3, 3), (1, 7, 2, 5), (64, 1, 1, 1), (130, 17, 0, 40)])
def test_dgrad_matches_the_decode_oracle(fmt, rows):
    N, K = 128, 128 if fmt == "nf4" else 96
    W, S = _stack(fmt, 4, N, K)
    sizes, ids = list(rows), [0, 1, 2, 3]
    go = rand_acts(sum(sizes), N, seed=2)
    got = dgrad = _ops()[fmt](go, W, S, sizes, ids)
    want = _oracle_bf16_path(fmt, go, W, S, [m for m in sizes], ids)
    assert got.shape == want.shape == (sum(sizes), K)
    assert rel_err(got, want) < 1e-2
    ref = _fp64(fmt, go, W, S, sizes, ids)
    e_f, e_d = rel_err(dgrad, ref), rel_err(want, ref)
    assert e_f <= 1e-2 and e_f <= 2 * e_d, (e_f, e_d)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_agrees_with_the_c_oracle_chain(fmt):
    N, K = 384, 512
    W, S = _stack(fmt, 5, N, K, seed=4)
    sizes, ids = [12, 1, 20, 70], [1, 3, 0, 4]
    go = rand_acts(sum(sizes), N, seed=5)
    got = _ops()[fmt](go, W, S, sizes, ids)
    ref = torch.from_numpy(oracle_dgrad(fmt, go, W, S, sizes, ids))
    assert rel_err(got.float().cpu(), ref) < 1e-2


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_one_hot_rows_are_exact(fmt):
    """grad row t one-hot at n = t selects decoded weight row t exactly."""
    N, K = 64, 256
    W, S = _stack(fmt, 2, N, K, seed=6)
    go = torch.eye(N, dtype=torch.bfloat16, device="cuda")
    for sizes in ([N], [1] * 4 + [N - 4]):
        ids = [1] * len(sizes)
        got = _ops()[fmt](go, W, S, sizes, ids)
        assert torch.equal(got, dequant(fmt, W[1], S[1]).to(torch.bfloat16))


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_output_does_not_depend_on_the_tile_config(fmt):
    N, K = 320, 384
    W, S = _stack(fmt, 4, N, K, seed=8)
    sizes, ids = [3, 1, 7, 2], [0, 1, 2, 3]
    go = rand_acts(sum(sizes), N, seed=9)
    op = _ops()[fmt]
    base = op(go, W, S, sizes, ids)
    for cfg in ((32, 64, 64, 2), (64, 64, 64, 4), (32, 128, 32, 2), (64, 32, 64, 8),
                (16, 64, 64, 2), (128, 64, 16, 4)):
        alt = op(go, W, S, sizes, ids, config=cfg)
        assert torch.equal(alt, base), f"config {cfg} changed the result"


def test_dgrad_eligibility_is_decidable_before_launching():
    from nf4_grouped import dgrad_4bit_grouped, dgrad_eligible
    W, S = rand_nf4_stack(4, 128, 128)
    go = rand_acts(13, 128)
    sizes, ids = [3, 1, 7, 2], [0, 1, 2, 3]
    assert dgrad_eligible(go, W, S) is None
    assert "bfloat16" in dgrad_eligible(go.to(torch.float16), W, S)
    assert "does not divide" in dgrad_eligible(go, W, S, block_k=48)
    with pytest.raises(ValueError, match="cannot run this problem"):
        dgrad_4bit_grouped(go.to(torch.float16), W, S, sizes, ids)


def test_dgrad_qwen_down_shape_contract():
    """Config-5 shape class (Qwen3 down, N=2048, K=768) at a reduced token count."""
    from nf4_grouped import dgrad_4bit_grouped
    E, N, K = 16, 2048, 768
    W, S = rand_nf4_stack(E, N, K, seed=10)
    sizes = [37, 128, 1, 300, 64, 0, 90, 5]
    ids = [0, 3, 5, 7, 9, 11, 13, 15]
    go = (rand_acts(sum(sizes), N, seed=11).float() * 1e-2).to(torch.bfloat16)
    got = dgrad_4bit_grouped(go, W, S, sizes, ids)
    ref = _fp64("nf4", go, W, S, sizes, ids)
    e_f = rel_err(got, ref)
    e_d = rel_err(_oracle_bf16_path("nf4", go, W, S, sizes, ids), ref)
    assert e_f <= 1e-2 and e_f <= 2 * e_d, (e_f, e_d)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_tall_tiles_and_k_tails(fmt):
    """Groups above 128 rows run 256-row tiles (the four-wave transposed-read
    kernel); K = 320 leaves one live 64-column block in the second 256-wide
    k tile."""
    N, K = 192, 320
    W, S = _stack(fmt, 6, N, K, seed=12)
    sizes, ids = [300, 129, 64, 1, 0, 200], [5, 0, 2, 3, 4, 1]
    go = rand_acts(sum(sizes), N, seed=13)
    got = _ops()[fmt](go, W, S, sizes, ids)
    want = _oracle_bf16_path(fmt, go, W, S, sizes, ids)
    assert rel_err(got, want) < 1e-2
    ref = _fp64(fmt, go, W, S, sizes, ids)
    e_f, e_d = rel_err(got, ref), rel_err(want, ref)
    assert e_f <= 1e-2 and e_f <= 2 * e_d, (e_f, e_d)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_tall_one_hot_rows_are_exact(fmt):
    """Every row of a 300-row group one-hot at n = t % N reproduces decoded
    row t % N bit for bit, through both 256-row tiles."""
    N, K, T = 128, 320, 300
    W, S = _stack(fmt, 2, N, K, seed=14)
    go = torch.zeros(T, N, dtype=torch.bfloat16, device="cuda")
    t = torch.arange(T, device="cuda")
    go[t, t % N] = 1
    got = _ops()[fmt](go, W, S, [T], [1])
    dec = dequant(fmt, W[1], S[1]).to(torch.bfloat16)
    assert torch.equal(got, dec[(t % N)])


def test_dgrad_tall_mxfp4_scale_extremes():
    """Small and large e8m0 exponents through the transposed-read kernel: each
    row of a block has its own scale, and one-hot rows give the decoded
    weights exactly, e8m0 0x00 (2^-127, subnormal weights) included."""
    N, K, T = 64, 128, 200
    W, S = rand_mx_stack(1, N, K, seed=15)
    S = S.clone()
    S[0, 1::5, 1] = 2
    S[0, 2::7, 3] = 140
    S[0, ::3, 0] = 0
    go = torch.zeros(T, N, dtype=torch.bfloat16, device="cuda")
    t = torch.arange(T, device="cuda")
    go[t, t % N] = 1
    got = _ops()["mxfp4"](go, W, S, [T], [0])
    want = dequant("mxfp4", W[0], S[0]).to(torch.bfloat16)[t % N]
    assert bool((S[0, :, 0] == 0).any())
    assert torch.equal(got, want)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_tall_several_tiles_per_workgroup(fmt):
    """40 groups of 300 one-hot rows x 4 output-column tiles: more tiles than
    the persistent grid has workgroups, so workgroups run several 256- and
    44-row tiles in turn. Row t of group g reproduces decoded row t % N of its
    expert bit for bit."""
    N, K, G, T = 128, 1024, 40, 300
    W, S = _stack(fmt, G, N, K, seed=16)
    ids = list(range(G - 1, -1, -1))
    go = torch.zeros(G * T, N, dtype=torch.bfloat16, device="cuda")
    t = torch.arange(G * T, device="cuda")
    go[t, (t % T) % N] = 1
    got = _ops()[fmt](go, W, S, [T] * G, ids)
    for g in (0, 1, G // 2, G - 1):
        dec = dequant(fmt, W[ids[g]], S[ids[g]]).to(torch.bfloat16)
        rows = torch.arange(T, device="cuda")
        assert torch.equal(got[g * T:(g + 1) * T], dec[rows % N]), g
