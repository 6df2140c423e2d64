"""Group-table staging of the launch paths on the GPU: the pinned table ring
read at its device address (decode launches), its copy fallback when the
host ring is not mapped for the device, and tables too large for a ring
part (to_device_i32's path). All must give the same bits."""
import pytest
import torch

import nf4_grouped
from _fixtures import rand_acts, rand_mx_stack, rand_nf4_stack

pytestmark = pytest.mark.gpu


def _ops():
    from mxfp4_grouped import gemm_mxfp4_grouped
    return {"nf4": (nf4_grouped.gemm_4bit_grouped, rand_nf4_stack),
            "mxfp4": (gemm_mxfp4_grouped, rand_mx_stack)}


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_unmapped_host_ring_copies_and_gives_the_same_bits(fmt):
    op, stack = _ops()[fmt]
    E, N, K = 16, 256, 512
    W, S = stack(E, N, K, seed=5)
    a = rand_acts(24, K, seed=6)
    cases = [([1] * 8, list(range(0, 16, 2))),            # one-row groups (decode)
             ([3, 1, 2, 4, 1, 5, 2, 6], list(range(8))),   # decode, several rows
             ([24], [7])]                                  # tiled path
    want = []
    for sizes, ids in cases:
        want.append(op(a[:sum(sizes)], W, S, sizes, ids))
    torch.cuda.synchronize()
    ring = nf4_grouped._table_ring(a.device, torch.cuda.current_stream())
    saved = ring.host_dev_ptr
    try:
        ring.host_dev_ptr = None                          # as if not mapped: copy
        for (sizes, ids), w in zip(cases, want):
            for _ in range(2):
                got = op(a[:sum(sizes)], W, S, sizes, ids)
                assert torch.equal(got.view(torch.int16), w.view(torch.int16)), sizes
    finally:
        ring.host_dev_ptr = saved


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_tables_larger_than_a_ring_part(fmt):
    """5000 one-row groups: expert ids and row offsets take 10001 ints, more
    than one part of the ring (8192), so the call uploads them on its own;
    its rows must be the bits of two calls of 2500 groups each."""
    op, stack = _ops()[fmt]
    E, N, K = 64, 64, 256
    W, S = stack(E, N, K, seed=8)
    G = 5000
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    sizes = [1] * G
    sizes[17] = 0                  # an empty group keeps a row-offset table
    T = sum(sizes)
    a = rand_acts(T, K, seed=10)
    assert 2 * G + 1 > nf4_grouped._TableRing.INTS // nf4_grouped._TableRing.PARTS
    whole = op(a, W, S, sizes, ids)
    h = G // 2
    t0 = sum(sizes[:h])
    first = op(a[:t0], W, S, sizes[:h], ids[:h])
    second = op(a[t0:], W, S, sizes[h:], ids[h:])
    assert torch.equal(whole.view(torch.int16), torch.cat([first, second]).view(torch.int16))
