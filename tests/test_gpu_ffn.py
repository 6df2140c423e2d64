"""GPU parity of the grouped NF4 expert FFN (gate_up -> silu(gate) * up -> down).

Bars:
  * silu-multiply: bit-exact against the locked fp32 spec (oracle/spec.py,
    the reference's kernel/cpu_grouped.py:147-179) on the bf16 gu values,
    clamps and tails included;
  * fused launch == gate_up forward -> silu-multiply -> down forward, bit for
    bit (the fusion moves where the chain runs, not what it computes; the
    reference's own bar for its fused CPU FFN, kernel/test_cpu_grouped.py:442-456);
  * against the reference's fp32 FFN (golden vectors written by its compiled
    CPU kernels, and the C oracle): within 1e-2 relative; against fp64 with
    the exact silu: B-abs <= 1e-2 and B-rel <= 2x a bf16 dequant-then-matmul
    composition.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from _fixtures import rand_acts, rand_nf4_stack, rel_err

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _mods():
    import nf4_ffn
    import nf4_grouped
    return nf4_ffn, nf4_grouped


def _stack(E, H, K, N_dn, seed=0, amax=(0.03, 0.08)):
    gu_p, gu_a = rand_nf4_stack(E, 2 * H, K, seed, amax_lo=amax[0], amax_hi=amax[1])
    dn_p, dn_a = rand_nf4_stack(E, N_dn, H, seed + 1)
    return gu_p, gu_a, dn_p, dn_a


def _composed(a, gu_p, gu_a, dn_p, dn_a, sizes, ids):
    nf4_ffn, nf4_grouped = _mods()
    gu = nf4_grouped.gemm_4bit_grouped(a, gu_p, gu_a, sizes, ids)
    h = nf4_ffn.silu_mul_locked(gu)
    return nf4_grouped.gemm_4bit_grouped(h, dn_p, dn_a, sizes, ids)


def _bits(x):
    return x.view(torch.int16)


# ---------------------------------------------------------- silu-multiply --

def test_silu_mul_is_bitwise_the_locked_spec():
    from oracle import spec
    nf4_ffn, _ = _mods()
    g = torch.Generator().manual_seed(7)
    T, H = 37, 512
    gu = torch.randn(T, 2 * H, generator=g) * 30
    gu[0, :8] = torch.tensor([87.0, -87.0, 87.5, -87.5, 300.0, -300.0, 0.0, -0.0])
    gu[1, :6] = torch.tensor([1e30, -1e30, 86.9, -86.9, 1e-20, -1e-20])
    gu = gu.to(torch.bfloat16)
    h = nf4_ffn.silu_mul_locked(gu.cuda()).cpu()
    gf = gu.float().numpy()
    want = spec.silu_locked(gf[:, :H]) * gf[:, H:]
    assert torch.equal(_bits(h), _bits(torch.from_numpy(want).to(torch.bfloat16)))


def test_silu_mul_strided_input_and_empty():
    nf4_ffn, _ = _mods()
    big = torch.randn(5, 400, device="cuda").to(torch.bfloat16)
    gu = big[:, :256]                                   # row stride 400
    h = nf4_ffn.silu_mul_locked(gu)
    assert torch.equal(_bits(h), _bits(nf4_ffn.silu_mul_locked(gu.contiguous())))
    assert nf4_ffn.silu_mul_locked(torch.zeros(0, 64, dtype=torch.bfloat16,
                                               device="cuda")).shape == (0, 32)


# ------------------------------------------------------- fused == composed --

QWEN = dict(E=128, H=768, K=2048, N_dn=2048)


@pytest.mark.parametrize("sizes,ids", [
    ([1] * 8, [3, 17, 40, 41, 77, 90, 101, 127]),      # B = 1, top-8
    ([2, 1, 3, 1, 16, 4], [0, 5, 9, 64, 100, 127]),    # ragged, one full 16-row group
    ([2, 2, 1], [7, 8, 9]),                            # staged activations (<= 2 rows)
    ([3, 0, 5, 0, 1], [1, 2, 3, 4, 5]),                # empty groups
])
def test_fused_equals_the_three_launch_composition_qwen3_shape(sizes, ids):
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(QWEN["E"], QWEN["H"], QWEN["K"], QWEN["N_dn"], seed=3)
    a = rand_acts(sum(sizes), QWEN["K"], seed=4)
    out = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
    ref = _composed(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)
    assert out.shape == (sum(sizes), QWEN["N_dn"]) and out.dtype == torch.bfloat16
    assert torch.equal(_bits(out), _bits(ref))
    assert not nf4_ffn.ffn_sync_error()


@pytest.mark.parametrize("H,K,N_dn", [(64, 64, 24), (128, 1024, 100), (256, 4096, 64),
                                      (2048, 512, 32)])
def test_fused_equals_composition_other_shapes(H, K, N_dn):
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(6, H, K, N_dn, seed=H + K)
    sizes, ids = [1, 4, 2, 1], [5, 0, 3, 1]
    a = rand_acts(sum(sizes), K, seed=5)
    out = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
    assert torch.equal(_bits(out), _bits(_composed(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)))


def test_expert_id_forms_and_repeats_are_bitwise_equal():
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(16, 256, 512, 128, seed=9)
    sizes, ids = [2, 1, 5], [11, 2, 7]
    a = rand_acts(sum(sizes), 512, seed=10)
    outs = [nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, e)
            for e in (ids, torch.tensor(ids), torch.tensor(ids, device="cuda"), ids, ids)]
    for o in outs[1:]:
        assert torch.equal(_bits(o), _bits(outs[0]))
    # the sync words are back at zero after every call
    for (_d, _s), buf in nf4_ffn._SYNC.items():
        assert int(buf.abs().sum().item()) == 0


def test_graph_replays_match_eager():
    """Capture the fused op once, replay it with eager work in between: the
    sync words must return to zero after every replay for the next to be
    right."""
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(32, 768, 2048, 2048, seed=12)
    sizes, ids = [1] * 8, [0, 3, 6, 9, 12, 15, 18, 21]
    a = rand_acts(8, 2048, seed=13)
    eager = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)   # warm-up
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(eager)), f"replay {i}"
        _ = (a.float() * 2).sum().item()                   # eager work between replays
    assert not nf4_ffn.ffn_sync_error()


# ------------------------------------------------- against the reference --

def _golden_cases():
    return sorted(GOLDEN.glob("ffn_*.npz"))


@pytest.mark.parametrize("path", _golden_cases(), ids=lambda p: p.stem)
def test_fused_against_the_reference_golden_vectors(path):
    """Inputs and fp32 outputs written by the reference's compiled CPU FFN."""
    nf4_ffn, _ = _mods()
    z = np.load(path)
    t = {k: torch.from_numpy(z[k]).cuda() for k in ("gu_packed", "gu_absmax", "dn_packed",
                                                    "dn_absmax")}
    a = torch.from_numpy(z["x"]).cuda()                  # fp32 activations: widened to bf16
    sizes, ids = z["sizes"].tolist(), z["eids"].tolist()
    out = nf4_ffn.gemm_nf4_ffn_grouped(a, t["gu_packed"], t["gu_absmax"], t["dn_packed"],
                                       t["dn_absmax"], sizes, ids)
    ref = torch.from_numpy(z["out"])
    assert rel_err(out.float().cpu(), ref) < 1e-2
    # the composition path agrees with the fused one on the same inputs
    comp = nf4_ffn.gemm_nf4_ffn_grouped(a, t["gu_packed"], t["gu_absmax"], t["dn_packed"],
                                        t["dn_absmax"], sizes, ids, fused=False)
    assert torch.equal(_bits(out), _bits(comp))


@pytest.mark.parametrize("sizes", [[1] * 8, [4, 9, 16, 2], [40, 3, 130]])
def test_contract_against_fp64_and_the_oracle(sizes):
    from oracle import native, spec
    nf4_ffn, nf4_grouped = _mods()
    E, H, K, N_dn = 8, 768, 2048, 2048
    gu_p, gu_a, dn_p, dn_a = _stack(E, H, K, N_dn, seed=21, amax=(0.2, 0.6))
    ids = list(range(len(sizes)))
    a = rand_acts(sum(sizes), K, seed=22)
    out = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)
    args = [x.cpu().numpy() for x in (gu_p, gu_a, dn_p, dn_a)]
    a32 = a.float().cpu().numpy()
    ref64 = torch.from_numpy(spec.fp64_ffn(a32, *args, sizes, ids))
    # bf16 dequant-then-matmul composition (the contract's comparator)
    outs, row = [], 0
    for m, e in zip(sizes, ids):
        wg = nf4_grouped.dequant_ref(gu_p[e], gu_a[e], 2 * H, K).to(torch.bfloat16)
        wd = nf4_grouped.dequant_ref(dn_p[e], dn_a[e], N_dn, H).to(torch.bfloat16)
        gu = (a[row:row + m] @ wg.t()).float()
        hh = (torch.nn.functional.silu(gu[:, :H]) * gu[:, H:]).to(torch.bfloat16)
        outs.append(hh @ wd.t())
        row += m
    e_f, e_d = rel_err(out.cpu(), ref64), rel_err(torch.cat(outs).cpu(), ref64)
    assert e_f <= 1e-2, f"B-abs {e_f:.3e}"
    assert e_f <= 2.0 * e_d, f"B-rel {e_f:.3e} > 2 x {e_d:.3e}"
    orc = torch.from_numpy(native.ffn_grouped(a32, *args, sizes, ids))
    assert rel_err(out.float().cpu(), orc) < 1e-2


# ---------------------------------------------------------------- errors --

def test_bad_calls_raise_like_the_reference():
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(4, 64, 128, 24, seed=30)
    a = rand_acts(3, 128, seed=31)
    sizes, ids = [1, 2], [0, 3]
    f = nf4_ffn.gemm_nf4_ffn_grouped
    with pytest.raises(ValueError, match="even"):
        f(a, gu_p[:, :-1], gu_a[:, :-1], dn_p, dn_a, sizes, ids)
    with pytest.raises(ValueError, match="H % 64"):
        f(a, gu_p[:, :64], gu_a[:, :64], dn_p, dn_a, sizes, ids)
    with pytest.raises(ValueError, match="expert counts"):
        f(a, gu_p, gu_a, dn_p[:2], dn_a[:2], sizes, ids)
    with pytest.raises(ValueError, match="out of range"):
        f(a, gu_p, gu_a, dn_p, dn_a, sizes, [0, 4])
    with pytest.raises(ValueError, match="at most 16"):
        f(rand_acts(17, 128, seed=32), gu_p, gu_a, dn_p, dn_a, [17], [0], fused=True)
    with pytest.raises(AssertionError):
        f(a, gu_p, gu_a, dn_p, dn_a, [1, 1], ids)


def test_decode_staging_bound_large_k():
    """Two-row groups with K large enough that staging their activations
    would exceed what the decode kernel's staging loop covers: they take the
    register path and still agree with the oracle."""
    from _fixtures import oracle_fwd
    from nf4_grouped import gemm_4bit_grouped
    K, N = 16384, 64
    W, S = rand_nf4_stack(3, N, K, seed=40)
    sizes, ids = [2, 2, 1], [2, 0, 1]
    a = rand_acts(5, K, seed=41)
    out = gemm_4bit_grouped(a, W, S, sizes, ids)
    ref = torch.from_numpy(oracle_fwd("nf4", a, W, S, sizes, ids))
    assert rel_err(out.float().cpu(), ref) < 1e-2


def test_many_groups_fused_and_auto_agree():
    """B = 16 routing (about 80 groups, above the auto threshold): the fused
    launch still gives the composition's bits, and the auto choice (the
    composition here) agrees."""
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(QWEN["E"], QWEN["H"], QWEN["K"], QWEN["N_dn"], seed=50)
    rng = np.random.default_rng(51)
    counts = np.zeros(QWEN["E"], np.int64)
    for _ in range(16):
        counts[rng.choice(QWEN["E"], 8, replace=False)] += 1
    ids = [int(e) for e in np.nonzero(counts)[0]]
    sizes = [int(counts[e]) for e in ids]
    assert nf4_ffn._fused_units(len(ids), QWEN["H"], QWEN["N_dn"]) > nf4_ffn.FUSED_MAX_UNITS
    a = rand_acts(sum(sizes), QWEN["K"], seed=52)
    fused = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
    auto = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)
    assert torch.equal(_bits(fused), _bits(auto))
    assert not nf4_ffn.ffn_sync_error()


# ------------------------------------------------------------ sync words --

def test_graph_of_a_smaller_call_survives_a_larger_capture():
    """Capture a fused call with one group, then one with many groups (it
    needs a larger sync buffer on the same capture stream), then replay the
    first graph with eager work in between: its sync words must still be its
    own (the outgrown buffer is kept alive), so both replays give the
    composition's bits and no error is raised."""
    nf4_ffn, nf4_grouped = _mods()
    H, K, N_dn, E = 256, 512, 384, 64
    gu_p, gu_a, dn_p, dn_a = _stack(E, H, K, N_dn, seed=60)
    dev = torch.device("cuda:0")
    cases = [([1], [5]), ([2, 1, 3, 1] * 12, list(range(0, 48)))]
    graphs, outs, wants = [], [], []
    for sizes, ids in cases:
        a = rand_acts(sum(sizes), K, seed=61 + len(sizes))
        plan = nf4_grouped.GroupPlan(sizes, ids, dev)
        wants.append(_composed(a, gu_p, gu_a, dn_p, dn_a, sizes, ids))
        out = torch.empty_like(wants[-1])
        h = torch.empty(a.shape[0], H, dtype=torch.bfloat16, device=dev)
        nf4_ffn.launch_ffn_planned(a, gu_p, gu_a, dn_p, dn_a, plan, h=h, out=out)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            nf4_ffn.launch_ffn_planned(a, gu_p, gu_a, dn_p, dn_a, plan, h=h, out=out)
        graphs.append((g, a, plan, h))
        outs.append(out)
    for rep in range(3):
        for (g, *_), out, want in zip(graphs, outs, wants):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            filler = torch.randn(1 << 20, device=dev)   # eager work between replays
            del filler
            assert torch.equal(_bits(out), _bits(want)), rep
    assert not nf4_ffn.ffn_sync_error()


def test_spin_expiry_poisons_the_rows_and_sets_the_error_word():
    """Force the time-out path from the host (a spin limit of 0 polls: a
    down unit that does not find its h ready at once gives up) -- every
    kernel still exits normally. Each down unit's output rows are then
    either the composition's bits or all NaN, the error word is set exactly
    when some are NaN, and after clearing it and restoring the limit the
    next call is exact again (no stale flag passes a later call)."""
    nf4_ffn, _ = _mods()
    H, K, N_dn, E = 512, 1024, 1024, 32
    gu_p, gu_a, dn_p, dn_a = _stack(E, H, K, N_dn, seed=70)
    sizes, ids = [1, 3, 2, 4, 1, 1, 2, 2], [3, 7, 11, 15, 19, 23, 27, 31]
    a = rand_acts(sum(sizes), K, seed=71)
    want = _composed(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)
    nf4_ffn.ffn_sync_clear()
    try:
        nf4_ffn.set_spin_limit(0)
        got = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
        torch.cuda.synchronize()
    finally:
        nf4_ffn.set_spin_limit(1 << 22)
    nan = torch.isnan(got.float())
    # a down unit covers 32 output columns of one group's rows
    row0 = 0
    for m in sizes:
        for c0 in range(0, N_dn, 32):
            blk = nan[row0:row0 + m, c0:c0 + 32]
            assert bool(blk.all()) or not bool(blk.any())
            if not bool(blk.any()):
                assert torch.equal(_bits(got[row0:row0 + m, c0:c0 + 32]),
                                   _bits(want[row0:row0 + m, c0:c0 + 32]))
        row0 += m
    timed_out = bool(nan.any())
    assert nf4_ffn.ffn_sync_error() == timed_out
    # flags the late gate/up units left behind carry the old call's epoch:
    # later calls wait for their own, so they are exact without a clear
    for _ in range(2):
        again = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
        assert torch.equal(_bits(again), _bits(want))
    assert nf4_ffn.ffn_sync_error() == timed_out     # sticky until cleared
    nf4_ffn.ffn_sync_clear()
    assert not nf4_ffn.ffn_sync_error()


@pytest.mark.parametrize("B", [1, 4])
def test_fused_hand_off_soak_in_graph_replays(B):
    """Bounded soak of the fused call at Qwen3-30B-A3B shapes -- batch 4: the
    single launch's cross-workgroup hand-off (gate/up units store h and then
    their flags with device-scope stores; down units on any XCD poll the
    flags and then load h); batch 1: its two-launch GEMV form -- 1500 replays
    of one captured call, the activations replaced before
    each replay from a pool of 12, every replay compared bit for bit with
    the three-launch composition of its activations; stops at the first
    mismatch."""
    nf4_ffn, nf4_grouped = _mods()
    q = QWEN
    gu_p, gu_a, dn_p, dn_a = _stack(q["E"], q["H"], q["K"], q["N_dn"], seed=140 + B)
    g = torch.Generator().manual_seed(141 + B)
    counts = torch.zeros(q["E"], dtype=torch.int64)
    for _ in range(B):
        counts[torch.randperm(q["E"], generator=g)[:8]] += 1
    ids = torch.nonzero(counts).flatten().tolist()
    sizes = counts[counts > 0].tolist()
    T = sum(sizes)
    pool = [rand_acts(T, q["K"], seed=150 + i) for i in range(12)]
    want = [_composed(x, gu_p, gu_a, dn_p, dn_a, sizes, ids) for x in pool]
    plan = nf4_grouped.GroupPlan(sizes, ids, "cuda")
    x = pool[0].clone()
    h = torch.empty(T, q["H"], dtype=torch.bfloat16, device="cuda")
    out = torch.empty(T, q["N_dn"], dtype=torch.bfloat16, device="cuda")
    nf4_ffn.launch_ffn_planned(x, gu_p, gu_a, dn_p, dn_a, plan, h=h, out=out)   # eager first
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        nf4_ffn.launch_ffn_planned(x, gu_p, gu_a, dn_p, dn_a, plan, h=h, out=out)
    for r in range(1500):
        i = (r * 7) % len(pool)
        x.copy_(pool[i])
        graph.replay()
        if not torch.equal(_bits(out), _bits(want[i])):
            pytest.fail(f"replay {r} (activations {i}) differs from the composition")
    assert not nf4_ffn.ffn_sync_error()


# ------------------------------------------- kernel-argument group tables --

@pytest.mark.parametrize("sizes", [
    [1] * 8,                 # batch 1, top-8: no offset table
    [2, 1, 2, 1],            # multi-row groups both stages' GEMVs take
    [1, 0, 1, 0, 1],         # empty groups (offset table, one-row GEMV)
])
def test_kernel_argument_tables_give_the_device_table_bits(sizes):
    nf4_ffn, nf4_grouped = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(QWEN["E"], QWEN["H"], QWEN["K"], QWEN["N_dn"], seed=21)
    G = len(sizes)
    ids = [(37 * g + 5) % QWEN["E"] for g in range(G)]
    a = rand_acts(sum(sizes), QWEN["K"], seed=22)
    ro = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    one_row = min(sizes) == 1 and max(sizes) == 1
    out = nf4_ffn._launch_fused_ids(a, gu_p, gu_a, dn_p, dn_a, np.asarray(ids, np.int32),
                                    None if one_row else ro, G, max(sizes))
    assert out is not None
    e_d = torch.tensor(ids, dtype=torch.int32, device="cuda")
    r_d = torch.from_numpy(ro).cuda()
    ref = nf4_ffn._launch_fused(a, gu_p, gu_a, dn_p, dn_a, e_d, r_d, G, max(sizes))
    assert torch.equal(_bits(out), _bits(ref))
    assert torch.equal(_bits(out), _bits(_composed(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)))


def test_kernel_argument_tables_refuse_before_launching():
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(QWEN["E"], QWEN["H"], QWEN["K"], QWEN["N_dn"], seed=23)
    # 3 rows: the down stage (K = 768) is no GEMV launch; the call returns
    # before launching, so the output buffer keeps its sentinel
    sizes, ids = [3, 1], [4, 9]
    a = rand_acts(4, QWEN["K"], seed=24)
    out = torch.full((4, QWEN["N_dn"]), 7.0, dtype=torch.bfloat16, device="cuda")
    ro = np.asarray([0, 3, 4], np.int32)
    assert nf4_ffn._launch_fused_ids(a, gu_p, gu_a, dn_p, dn_a, np.asarray(ids, np.int32), ro,
                                     2, 3, out=out) is None
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    # the op then takes the device-table launch: same bits as the chain
    got = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
    assert torch.equal(_bits(got), _bits(_composed(a, gu_p, gu_a, dn_p, dn_a, sizes, ids)))


@pytest.mark.parametrize("G", [384, 385])
def test_kernel_argument_tables_at_and_past_their_size(G):
    nf4_ffn, _ = _mods()
    E, H, K, N_dn = 16, 64, 128, 64
    gu_p, gu_a, dn_p, dn_a = _stack(E, H, K, N_dn, seed=25)
    sizes, ids = [1] * G, [(7 * g) % E for g in range(G)]
    a = rand_acts(G, K, seed=26)
    got = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
    dev_ids = torch.tensor(ids, device="cuda")
    ref = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, dev_ids, fused=True)
    assert torch.equal(_bits(got), _bits(ref))


def test_kernel_argument_tables_planned_in_a_graph():
    nf4_ffn, nf4_grouped = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(QWEN["E"], QWEN["H"], QWEN["K"], QWEN["N_dn"], seed=27)
    sizes, ids = [1] * 8, [3, 17, 40, 41, 77, 90, 101, 127]
    a = rand_acts(8, QWEN["K"], seed=28)
    plan = nf4_grouped.GroupPlan(sizes, ids, "cuda")
    h = torch.empty(8, QWEN["H"], dtype=torch.bfloat16, device="cuda")
    out = torch.empty(8, QWEN["N_dn"], dtype=torch.bfloat16, device="cuda")
    want = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes,
                                        torch.tensor(ids, device="cuda"), fused=True)
    nf4_ffn.launch_ffn_planned(a, gu_p, gu_a, dn_p, dn_a, plan, h=h, out=out)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(want))
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            nf4_ffn.launch_ffn_planned(a, gu_p, gu_a, dn_p, dn_a, plan, h=h, out=out)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_bits(out), _bits(want))


def test_kernel_argument_tables_reject_bad_ids():
    nf4_ffn, _ = _mods()
    gu_p, gu_a, dn_p, dn_a = _stack(8, 64, 128, 64, seed=29)
    a = rand_acts(2, 128, seed=30)
    with pytest.raises(ValueError):
        nf4_ffn._launch_fused_ids(a, gu_p, gu_a, dn_p, dn_a, np.asarray([1, -1], np.int32),
                                  None, 2, 1)
    with pytest.raises(ValueError):   # decreasing offsets
        nf4_ffn._launch_fused_ids(a, gu_p, gu_a, dn_p, dn_a, np.asarray([1, 2], np.int32),
                                  np.asarray([0, 2, 1], np.int32), 2, 1)
