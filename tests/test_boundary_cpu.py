"""Host-side behaviour of the drop-in boundary, checked without a GPU.

Mirrors the reference's device-free tests: plan KATs
(kernel/test_nf4_grouped.py:209-245, :305-309), tile-table semantics
(kernel/test_group_tiles_readonly.py:25-49), CPU refusal text
(kernel/test_cpu_refusal.py:17-32), dgrad eligibility
(kernel/test_nf4_grouped.py:386-400) and the argument contract.
"""
import pytest
import torch

import mxfp4_grouped
import nf4_grouped
from nf4_grouped import (_decode_plan, _prefill_block_m, _tiles_host, build_group_tiles,
                         decode_dispatch, dgrad_4bit_grouped, dgrad_eligible, gemm_4bit_grouped,
                         to_device_i32)


# ------------------------------------------------------------------- plans --

def test_prefill_block_m_rule():
    assert [_prefill_block_m(m) for m in (1, 16, 17, 32, 33, 64, 65, 128, 256)] == \
        [16, 16, 32, 32, 64, 64, 128, 128, 128]


def test_decode_plan_thresholds():
    for sm in (26, 64):
        bn, w, _ = _decode_plan(2048, 768, 8, sm)
        assert (bn, w) == (64, 2)
    assert _decode_plan(5120, 8192, 1, 64) == (64, 2, 4)
    for N, K in ((2048, 2048), (1408, 2816), (1536, 2048), (2880, 2880)):
        for sm in (26, 64):
            assert _decode_plan(N, K, 8, sm)[2] == 1
    assert _decode_plan(64, 64, 1, 64)[2] == 1
    assert _decode_plan(6144, 768, 1, 64)[2] == 1
    assert _decode_plan(64, 8192, 1, 64)[2] == 4


def test_decode_dispatch_floor():
    assert decode_dispatch(6144, 768, 1, 64) == ("dequant",)
    assert decode_dispatch(768, 3072, 1, 64) == ("dequant",)
    d = decode_dispatch(1536, 512, 8, 64)
    assert d[0] == "fused" and d[1:3] == (64, 2)
    assert decode_dispatch(2048, 2048, 8, 64) == ("fused", 64, 2, 1)
    assert decode_dispatch(5120, 8192, 1, 64) == ("fused", 64, 2, 4)


def test_exported_constants():
    assert nf4_grouped.DECODE_MIN_FUSED_BYTES == 3_000_000
    assert nf4_grouped.SPLITK_MIN_BLOCKS == 32
    assert nf4_grouped._DGRAD_DEFAULT == (32, 64, 64, 2)
    assert nf4_grouped.HAS_TL_GATHER is True
    assert nf4_grouped._sm_count("cpu") == 64
    assert nf4_grouped._lut("cpu").tolist() == nf4_grouped.NF4_LUT
    assert mxfp4_grouped._lut("cpu").tolist() == mxfp4_grouped.FP4_VALUES
    assert mxfp4_grouped._prefill_block_m is nf4_grouped._prefill_block_m
    assert mxfp4_grouped.build_group_tiles is nf4_grouped.build_group_tiles


# ------------------------------------------------------------ tile tables --

def _tiles_brute(sizes, bm):
    out = []
    row = 0
    for g, m in enumerate(sizes):
        for r in range(0, m, bm):
            out.append((row + r, min(bm, m - r), g))
        row += m
    return out


@pytest.mark.parametrize("sizes", [[1], [16, 17, 0, 3], [128, 129, 1], [0, 0], [5, 300, 64]])
@pytest.mark.parametrize("bm", [16, 32, 64, 128])
def test_tiles_closed_form(sizes, bm):
    t0, tr, tg = _tiles_host(sizes, bm)
    assert list(zip(t0, tr, tg)) == _tiles_brute(sizes, bm)
    assert sum(tr) == sum(sizes)
    assert all(0 < r <= bm for r in tr)


def test_build_group_tiles_reads_sizes_only():
    sizes = torch.tensor([40, 0, 25])
    a = build_group_tiles(sizes, 16, "cpu")
    b = build_group_tiles(sizes, 16, "cpu")
    assert sizes.tolist() == [40, 0, 25]
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    c = build_group_tiles([40, 0, 25], 16, "cpu")
    assert all(torch.equal(x, y) for x, y in zip(a, c))
    assert a[0].dtype == torch.int32 and a[0].tolist() == [0, 16, 32, 40, 56]
    assert a[1].tolist() == [16, 16, 8, 16, 9] and a[2].tolist() == [0, 0, 0, 2, 2]


def test_to_device_i32_values_and_forms():
    outs = to_device_i32(([3, 1, 2], torch.tensor([7, 8]), []), "cpu")
    assert [o.tolist() for o in outs] == [[3, 1, 2], [7, 8], []]
    assert all(o.dtype == torch.int32 for o in outs)
    assert [o.numel() for o in to_device_i32(([], []), "cpu")] == [0, 0]


# ------------------------------------------------------------- refusals --

def _cpu_case():
    E, N, K = 2, 32, 64
    B = torch.zeros(E, N, K // 2, dtype=torch.uint8)
    A = torch.ones(E, N, K // 64)
    a = torch.zeros(3, K, dtype=torch.bfloat16)
    return a, B, A


def test_cpu_tensors_are_refused_with_the_reference_message():
    a, B, A = _cpu_case()
    with pytest.raises(RuntimeError) as ei:
        gemm_4bit_grouped(a, B, A, [2, 1], [0, 1])
    msg = str(ei.value).lower()
    assert "cuda" in msg and "dequant_ref" in msg
    with pytest.raises(RuntimeError) as ei:
        dgrad_4bit_grouped(torch.zeros(3, 32, dtype=torch.bfloat16), B, A, [2, 1], [0, 1])
    assert "cuda" in str(ei.value).lower() and "dequant_ref" in str(ei.value)
    S = torch.zeros(2, 32, 2, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="(?i)cuda"):
        mxfp4_grouped.gemm_mxfp4_grouped(a, B, S, [2, 1], [0, 1])


def test_size_mismatch_is_an_assertion_before_anything_else():
    a, B, A = _cpu_case()
    with pytest.raises(AssertionError):
        gemm_4bit_grouped(a, B, A, [2, 2], [0, 1])
    with pytest.raises(AssertionError):
        dgrad_4bit_grouped(torch.zeros(3, 32, dtype=torch.bfloat16), B, A, [1, 1], [0, 1])
    S = torch.zeros(2, 32, 2, dtype=torch.uint8)
    with pytest.raises(AssertionError):
        mxfp4_grouped.gemm_mxfp4_grouped(a, B, S, [1, 1], [0, 1])
    with pytest.raises(AssertionError):
        mxfp4_grouped.gemm_mxfp4_grouped(a, B, S[:, :, :1], [2, 1], [0, 1])


def test_dgrad_eligibility_reasons():
    _, B, A = _cpu_case()
    go = torch.zeros(3, 32, dtype=torch.bfloat16)
    assert dgrad_eligible(go, B, A) is None
    assert "bfloat16" in dgrad_eligible(go.to(torch.float16), B, A)
    assert "does not divide" in dgrad_eligible(go, B, A, block_k=48)
    assert "do not tile" in dgrad_eligible(go, B, A[:, :, :0])
    assert "empty" in dgrad_eligible(go, B[:, :0], A[:, :0])


def test_dequant_ref_runs_on_cpu():
    B = torch.full((1, 32), 0x77, dtype=torch.uint8)      # code 7 = 0.0
    B[0, 0], B[0, 1] = 0x7F, 0xF0
    A = torch.tensor([[2.0]])
    w = nf4_grouped.dequant_ref(B, A, 1, 64)
    assert w[0, :4].tolist() == [0.0, 2.0, 2.0, -2.0] and not w[0, 4:].any()


def test_op_modules_do_not_import_the_oracle():
    """The product path never routes through the checker."""
    import ast
    import inspect
    for mod in (nf4_grouped, mxfp4_grouped, __import__("_hiplib"), __import__("nf4_qlora")):
        tree = ast.parse(inspect.getsource(mod))
        names = set()
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                names |= {a.name for a in node.names}
            elif isinstance(node, ast.ImportFrom):
                names.add(node.module or "")
        assert not any(n.split(".")[0] == "oracle" for n in names), (mod.__name__, names)


def test_numpy_tile_tables_equal_the_reference_tiling():
    """The launch paths' numpy tile tables equal the list tiling (the
    reference's build_group_tiles order), and the XCD ordering is the same
    permutation on both forms."""
    import numpy as np
    from nf4_grouped import _tiles_host, _tiles_np, _xcd_balanced
    rng = np.random.default_rng(5)
    for trial in range(40):
        G = int(rng.integers(0, 60))
        sizes = [int(v) for v in rng.integers(0, 700, G)]
        if trial % 5 == 0 and G:
            sizes[0] = 0
        for bm in (16, 32, 64, 128, 256):
            ref = _tiles_host(sizes, bm)
            got = _tiles_np(sizes, bm)
            assert all(g.dtype == np.int32 for g in got)
            assert [g.tolist() for g in got] == [list(r) for r in ref]
            if bm == 256:
                a = _xcd_balanced(*ref)
                b = _xcd_balanced(*got)
                assert [list(x) for x in a] == [y.tolist() for y in b]


def test_ring_registry_gives_every_thread_the_same_object():
    """Two threads making their first call on one stream must share its
    staging ring (a dropped ring's pinned block could be reused while a
    kernel still reads group tables from it): creation runs under a lock and
    re-checks the table."""
    import threading
    table, made = {}, []
    gate = threading.Barrier(8)

    def make():
        made.append(object())
        return made[-1]

    got = []

    def worker():
        gate.wait()
        got.append(nf4_grouped._registered(table, ("cuda:0", 1234), make))

    ts = [threading.Thread(target=worker) for _ in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert len(made) == 1 and all(g is made[0] for g in got) and table[("cuda:0", 1234)] is made[0]
