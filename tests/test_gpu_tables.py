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


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("ids_on", ["host", "device"])
def test_kernel_argument_tile_tables_give_the_same_bits(fmt, ids_on, monkeypatch):
    """256-row tiled calls whose table fits the kernel arguments (no upload)
    against the same calls with the table uploaded (ARG_TILES_MAX = 0):
    bitwise, with host and device expert ids, ragged groups (empty, 1, 255,
    256, 257, 700 rows)."""
    op, stack = _ops()[fmt]
    E, N, K = 64, 544, 1024
    W, S = stack(E, N, K, seed=21)
    sizes = [300, 0, 1, 255, 256, 257, 700, 40]
    ids = [5, 9, 0, 63, 17, 2, 40, 33]
    T = sum(sizes)
    a = rand_acts(T, K, seed=22)
    eids = torch.tensor(ids, dtype=torch.int32, device="cuda") if ids_on == "device" else ids
    got = op(a, W, S, sizes, eids)
    monkeypatch.setattr(nf4_grouped, "ARG_TILES_MAX", 0)
    want = op(a, W, S, sizes, eids)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("ids_on", ["host", "device"])
def test_kernel_argument_tile_tables_dgrad(fmt, ids_on, monkeypatch):
    """dgrad on 256-row tiles: kernel-argument table against the uploaded
    one, bitwise."""
    from mxfp4_grouped import dgrad_mxfp4_grouped
    dg = nf4_grouped.dgrad_4bit_grouped if fmt == "nf4" else dgrad_mxfp4_grouped
    _, stack = _ops()[fmt]
    E, N, K = 32, 512, 768
    W, S = stack(E, N, K, seed=23)
    sizes = [129, 256, 0, 400, 3, 200]
    ids = [31, 0, 7, 12, 30, 5]
    go = (rand_acts(sum(sizes), N, seed=24).float() * 1e-2).to(torch.bfloat16)
    eids = torch.tensor(ids, dtype=torch.int32, device="cuda") if ids_on == "device" else ids
    got = dg(go, W, S, sizes, eids)
    monkeypatch.setattr(nf4_grouped, "ARG_TILES_MAX", 0)
    want = dg(go, W, S, sizes, eids)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_more_tiles_than_the_kernel_arguments_hold():
    """300 groups of 200 rows: 300 m-tiles, more than the kernel-argument
    table holds, so the call uploads the table; rows of a few groups against
    single-group calls, bitwise."""
    op, stack = _ops()["nf4"]
    E, N, K = 8, 256, 1024
    W, S = stack(E, N, K, seed=25)
    G = 300
    sizes = [200] * G
    ids = [i % E for i in range(G)]
    a = rand_acts(sum(sizes), K, seed=26)
    assert G > nf4_grouped.ARG_TILES_MAX
    got = op(a, W, S, sizes, ids)
    for g in (0, 1, 150, 299):
        r0 = 200 * g
        one = op(a[r0:r0 + 200], W, S, [200], [ids[g]])
        assert torch.equal(got[r0:r0 + 200].view(torch.int16), one.view(torch.int16)), g


def test_kernel_argument_tables_in_graph_replays():
    """A captured 256-row tiled call (kernel-argument table, so the graph has
    no copy node) replayed with fresh activations: every replay equals the
    eager call on the same activations."""
    op, stack = _ops()["nf4"]
    E, N, K = 16, 512, 1024
    W, S = stack(E, N, K, seed=27)
    sizes, ids = [300, 260, 0, 512], [3, 15, 8, 0]
    a = rand_acts(sum(sizes), K, seed=28)
    op(a, W, S, sizes, ids)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        op(a, W, S, sizes, ids)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            out = op(a, W, S, sizes, ids)
    torch.cuda.current_stream().wait_stream(s)
    for r in range(4):
        a.copy_(rand_acts(sum(sizes), K, seed=40 + r))
        graph.replay()
        torch.cuda.synchronize()
        want = op(a, W, S, sizes, ids)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), r


@pytest.mark.parametrize("fmt,K,sizes", [
    ("nf4", 2048, [1] * 8), ("nf4", 768, [1] * 8), ("nf4", 2048, [1, 3, 2, 0, 4, 1]),
    ("nf4", 768, [2, 1, 2, 1]), ("mxfp4", 2880, [1] * 4), ("nf4", 2048, [1, 8, 2]),
])
def test_kernel_argument_expert_ids_give_the_same_bits(fmt, K, sizes, monkeypatch):
    """Decode calls with host ids pass them in the GEMV kernels' arguments;
    the same calls with device ids (a table the kernel reads) and with the
    argument path switched off give the same bits. The last case has a
    group of 8 rows, which no GEMV class takes: it falls back to the tables."""
    op, stack = _ops()[fmt]
    E, N = 32, 320
    W, S = stack(E, N, K, seed=31)
    ids = [(7 * g + 3) % E for g in range(len(sizes))]
    a = rand_acts(sum(sizes), K, seed=32)
    got = op(a, W, S, sizes, ids)
    dev_ids = op(a, W, S, sizes, torch.tensor(ids, dtype=torch.int32, device="cuda"))
    monkeypatch.setattr(nf4_grouped, "IDS_ARG_MAX", 0)
    want = op(a, W, S, sizes, ids)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(dev_ids.view(torch.int16), want.view(torch.int16))


def test_kernel_argument_expert_ids_planned_and_many_groups(monkeypatch):
    """launch_planned with host ids in the kernel arguments against the
    device tables; and 400 one-row groups (more than the arguments hold),
    which upload the tables: rows against single-group calls."""
    op, stack = _ops()["nf4"]
    E, N, K = 16, 256, 1024
    W, S = stack(E, N, K, seed=33)
    sizes, ids = [1, 2, 1, 1], [4, 15, 0, 9]
    a = rand_acts(sum(sizes), K, seed=34)
    plan = nf4_grouped.GroupPlan(sizes, ids, a.device)
    got = nf4_grouped.launch_planned(0, a, W, S, plan)
    monkeypatch.setattr(nf4_grouped, "IDS_ARG_MAX", 0)
    want = nf4_grouped.launch_planned(0, a, W, S, plan)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    monkeypatch.undo()
    G = 400
    ids = [g % E for g in range(G)]
    a = rand_acts(G, K, seed=35)
    assert G > nf4_grouped.IDS_ARG_MAX
    got = op(a, W, S, [1] * G, ids)
    for g in (0, 7, 399):
        one = op(a[g:g + 1], W, S, [1], [ids[g]])
        assert torch.equal(got[g].view(torch.int16), one[0].view(torch.int16)), g


# ---------------------------------------------- (first, end) row-pair tables --

def _pairs_call(fmt, a, W, S, ids_dev, pairs_dev, G, max_m, out):
    import _hiplib
    W, S = nf4_grouped._aligned_rows(W, 16), nf4_grouped._scales_view(S)
    rc = _hiplib.load().gnf4_hip_grouped_decode_pairs(
        0 if fmt == "nf4" else 1, a.data_ptr(), _hiplib.DTYPE_BF16, a.stride(0),
        W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
        ids_dev.data_ptr(), pairs_dev.data_ptr(), G, max_m, W.shape[1], a.shape[1],
        out.data_ptr(), out.stride(0), torch.cuda.current_stream().cuda_stream)
    _hiplib.check(rc, "decode_pairs")


@pytest.mark.parametrize("fmt,N,K,hi", [("nf4", 2048, 768, 3), ("nf4", 1536, 2048, 9),
                                        ("nf4", 256, 512, 16), ("mxfp4", 640, 1440, 5),
                                        ("mxfp4", 256, 2880, 1)])
def test_row_pairs_in_any_order_give_the_prefix_table_bits(fmt, N, K, hi):
    """Groups listed in a random order as (first, end) row pairs: every row
    is the bits of the prefix-offset launch of the same groups (the device
    id form, which keeps the groups in row order). Empty groups included."""
    op, stack = _ops()[fmt]
    E, G = 20, 37
    W, S = stack(E, N, K, seed=40)
    g = torch.Generator().manual_seed(41)
    sizes = torch.randint(0, hi + 1, (G,), generator=g).tolist()
    sizes[0], sizes[5] = hi, 0
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    T = sum(sizes)
    a = rand_acts(T, K, seed=42)
    want = op(a, W, S, sizes, torch.tensor(ids, device="cuda"))
    first = [sum(sizes[:i]) for i in range(G)]
    perm = torch.randperm(G, generator=g).tolist()
    pairs = [v for i in perm for v in (first[i], first[i] + sizes[i])]
    out = torch.full((T, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _pairs_call(fmt, a, W, S, torch.tensor([ids[i] for i in perm], dtype=torch.int32,
                                           device="cuda"),
                torch.tensor(pairs, dtype=torch.int32, device="cuda"), G, max(sizes), out)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    # the op with host ids (largest first) and the planned launch agree
    got = op(a, W, S, sizes, ids)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    plan = nf4_grouped.GroupPlan(sizes, ids, "cuda")
    assert plan.row_pairs is not None
    planned = nf4_grouped.launch_planned(0 if fmt == "nf4" else 1, a, W, S, plan)
    assert torch.equal(planned.view(torch.int16), want.view(torch.int16))


def test_row_pairs_past_65535_groups():
    """70000 groups of one or two rows as row pairs, largest first: the
    launch runs as several grid ranges (each taking its slice of the pair
    table); the bits are those of the prefix-offset launch."""
    op, stack = _ops()["nf4"]
    E, N, K, G = 4, 32, 128, 70000
    W, S = stack(E, N, K, seed=43)
    g = torch.Generator().manual_seed(44)
    sizes = (1 + (torch.rand(G, generator=g) < 0.1).int()).tolist()
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    a = rand_acts(sum(sizes), K, seed=45)
    want = op(a, W, S, sizes, torch.tensor(ids, device="cuda"))
    got = op(a, W, S, sizes, ids)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_row_pair_tables_reject_bad_arguments():
    import _hiplib
    lib = _hiplib.load()
    W, S = rand_nf4_stack(2, 64, 128, seed=46)
    a = rand_acts(4, 128, seed=47)
    out = torch.empty(4, 64, dtype=torch.bfloat16, device="cuda")
    ids = torch.zeros(2, dtype=torch.int32, device="cuda")
    pairs = torch.tensor([0, 2, 2, 4], dtype=torch.int32, device="cuda")
    for max_m, p in ((0, pairs), (17, pairs), (2, None)):
        rc = lib.gnf4_hip_grouped_decode_pairs(
            0, a.data_ptr(), _hiplib.DTYPE_BF16, a.stride(0), W.data_ptr(), W.stride(0),
            W.stride(1), S.data_ptr(), S.stride(0), S.stride(1), ids.data_ptr(),
            p.data_ptr() if p is not None else None, 2, max_m, 64, 128, out.data_ptr(),
            out.stride(0), torch.cuda.current_stream().cuda_stream)
        assert rc == -1
