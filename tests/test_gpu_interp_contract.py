"""The reference's device-free contract and fuzz suite, restated on the GPU.

kernel/test_interp_contract.py:46-109 runs the Triton kernels under the
interpreter on boundary shapes -- decode and prefill against dequant_ref of
the same bytes, N not a multiple of the block, one group, many groups of one
expert, K == BLOCKSIZE, random shapes from a seeded generator, one absmax
block with a 1e3 outlier -- with the bar
max|out - ref| / max|ref| < 1e-2 against an fp32 reference (:45). The same
shapes run here through the HIP kernels, NF4 and MXFP4, with that bar and
the tolerance contract's (B-abs and B-rel against fp64, `contract_check`).
The fuzz draws more cases than the reference's six and lets some groups
exceed 128 rows, so every kernel family of the dispatch is reached.
"""
import pytest
import torch

from _fixtures import contract_check, fp64_ref, rand_acts, rand_mx_stack, rand_nf4_stack

pytestmark = pytest.mark.gpu


def _ops(fmt):
    if fmt == "nf4":
        from nf4_grouped import gemm_4bit_grouped
        return gemm_4bit_grouped
    from mxfp4_grouped import gemm_mxfp4_grouped
    return gemm_mxfp4_grouped


def _stack(fmt, E, N, K, seed):
    return rand_nf4_stack(E, N, K, seed) if fmt == "nf4" else rand_mx_stack(E, N, K, seed)


def _max_rel(out, ref):
    """The reference's bar: max abs error over max abs reference (:45)."""
    return ((out.double() - ref).abs().max() / ref.abs().max().clamp_min(1e-4)).item()


def _run(fmt, E, N, K, sizes, ids, seed=0):
    W, S = _stack(fmt, E, N, K, seed)
    a = rand_acts(sum(sizes), K, seed=seed + 1)
    out = _ops(fmt)(a, W, S, sizes, torch.tensor(ids, dtype=torch.int32))
    assert out.shape == (sum(sizes), N) and out.dtype == torch.bfloat16
    ref = fp64_ref(fmt, a, W, S, sizes, ids)
    assert _max_rel(out, ref) < 1e-2, (fmt, E, N, K, sizes, ids)
    contract_check(fmt, out, a, W, S, sizes, ids)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("N,K", [(32, 128), (128, 256), (48, 64), (2048, 128)])
def test_decode_matches_reference(fmt, N, K):
    _run(fmt, 4, N, K, [1, 1, 1], [1, 3, 0])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("m", [4, 16, 65])
def test_prefill_matches_reference(fmt, m):
    _run(fmt, 4, 128, 128, [m, 1], [2, 0])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("sizes", [[1, 1], [5, 40]])
def test_n_not_a_multiple_of_the_block(fmt, sizes):
    # N = 130: a ragged last weight-row tile, and not a multiple of 4 (the
    # tiled call takes the fallback kernel)
    _run(fmt, 3, 130, 128, sizes, [0, 2])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_single_group(fmt):
    _run(fmt, 2, 64, 64, [1], [1])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("m", [1, 7])
def test_many_groups_same_expert(fmt, m):
    # 12 groups, all on expert 0: the expert's weights feed every group
    _run(fmt, 2, 96, 128, [m] * 12, [0] * 12)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_min_k(fmt):
    # K == BLOCKSIZE (NF4); MXFP4 takes its own block, K == 32
    _run(fmt, 2, 64, 64 if fmt == "nf4" else 32, [1, 1], [0, 1])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("seed", range(16))
def test_fuzz_random_shapes(fmt, seed):
    g = torch.Generator().manual_seed(1000 * (fmt == "mxfp4") + seed)
    blk = 64 if fmt == "nf4" else 32
    E = int(torch.randint(1, 6, (1,), generator=g))
    N = int(torch.randint(1, 40, (1,), generator=g)) * 8          # 8..312
    K = int(torch.randint(1, 9, (1,), generator=g)) * blk         # up to 512 / 256
    G = int(torch.randint(1, 6, (1,), generator=g))
    big = seed % 4 == 3     # every fourth case: groups up to 300 rows
    hi = 301 if big else 4
    sizes = [int(torch.randint(1, hi, (1,), generator=g)) for _ in range(G)]
    ids = [int(torch.randint(0, E, (1,), generator=g)) for _ in range(G)]
    _run(fmt, E, N, K, sizes, ids, seed=seed)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_adversarial_block_outlier(fmt):
    # one scale block of expert 0 a thousand times the rest (MXFP4: +10 in
    # the e8m0 exponent, 1024x)
    W, S = _stack(fmt, 2, 64, 128, seed=7)
    if fmt == "nf4":
        S[0, :, 0] *= 1e3
    else:
        S[0, :, 0] += 10
    a = rand_acts(1, 128, seed=8)
    out = _ops(fmt)(a, W, S, [1], torch.tensor([0], dtype=torch.int32))
    ref = fp64_ref(fmt, a, W, S, [1], [0])
    assert _max_rel(out, ref) < 1e-2
    contract_check(fmt, out, a, W, S, [1], [0])
