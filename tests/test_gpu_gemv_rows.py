"""GPU parity of the multi-row NF4 decode GEMV (groups of 2..4 rows, K <= 2048).

Such launches run k_gemv_nf4 as one-row passes over each group, so every
output row must be the same bits as that row computed as a one-row group
(the one-row summation order, which the C oracle's locked tree does not
share: against it and against fp64 the bar is the tolerance contract). The
fused FFN's GEMV form must equal gate_up forward -> silu-multiply -> down
forward bit for bit, including the mixed case where only the down stage is
a GEMV (gate_up K > 2048).
"""
import pytest
import torch

from _fixtures import contract_check, oracle_fwd, rand_acts, rand_nf4_stack, rel_err

pytestmark = pytest.mark.gpu


def _op():
    from nf4_grouped import gemm_4bit_grouped
    return gemm_4bit_grouped


def _one_row_groups(sizes, ids):
    rid = [i for i, m in enumerate(sizes) for _ in range(m)]
    return [1] * len(rid), [ids[i] for i in rid]


@pytest.mark.parametrize("N,K,rows,G", [(1536, 2048, 4, 60), (2048, 768, 2, 60), (640, 1024, 2, 40),
                                        (200, 512, 2, 30), (96, 64, 2, 9), (1000, 1344, 4, 25),
                                        (1530, 2048, 4, 3), (700, 1088, 3, 20)])
def test_multi_row_groups_give_the_bits_of_one_row_groups(N, K, rows, G):
    """Ragged groups of 0..rows rows (one of exactly `rows`; the class takes
    up to 4 rows at 1024 < K <= 2048, up to 2 at K <= 1024), N off the
    row-step multiple (1000, 1530, 200, 700), K from one absmax block pair
    (64) to 2048 and between (1344, 1088: a partial last slot round)."""
    E = 24
    W, S = rand_nf4_stack(E, N, K, seed=N + K)
    g = torch.Generator().manual_seed(rows * 1000 + G)
    sizes = torch.randint(0, rows + 1, (G,), generator=g).tolist()
    sizes[G // 2] = rows
    sizes[0] = 0
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    a = rand_acts(sum(sizes), K, seed=5)
    op = _op()
    out = op(a, W, S, sizes, ids)
    s1, i1 = _one_row_groups(sizes, ids)
    assert torch.equal(out, op(a, W, S, s1, i1))
    sel = list(range(0, sum(sizes), 3))
    contract_check("nf4", out[sel], a[sel], W, S, [1] * len(sel), [i1[r] for r in sel])


def test_multi_row_gemv_agrees_with_the_c_oracle():
    E, N, K = 6, 320, 1024
    W, S = rand_nf4_stack(E, N, K, seed=3)
    sizes, ids = [3, 0, 4, 1, 2], [5, 1, 0, 0, 3]
    a = rand_acts(sum(sizes), K, seed=4)
    out = _op()(a, W, S, sizes, ids)
    ref = oracle_fwd("nf4", a, W, S, sizes, ids)
    assert rel_err(out, torch.from_numpy(ref).to(out.device)) <= 1e-2


def test_device_routed_plan_of_four_tokens_takes_the_gemv_class():
    """A device-routed decode of T = 4 tokens passes max_m = 4: at K = 2048
    the launch is the GEMV class, so each token's expert rows are the bits
    of that token alone (T = 1)."""
    import nf4_route
    E, N, K, k, T = 16, 512, 2048, 4, 4
    W, S = rand_nf4_stack(E, N, K, seed=9)
    x = rand_acts(T, K, seed=10)
    g = torch.Generator().manual_seed(11)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    ids[1] = ids[0]                       # two tokens share all four experts
    ids = ids.cuda()
    plan = nf4_route.route_groups(ids, E)
    a = nf4_route.gather_rows(x, plan)
    y = nf4_route._decode_fwd(a, W, S, plan, T)
    for t in range(T):
        p1 = nf4_route.route_groups(ids[t:t + 1], E)
        y1 = nf4_route._decode_fwd(nf4_route.gather_rows(x[t:t + 1], p1), W, S, p1, 1)
        got = nf4_route.combine(y, plan, torch.ones(T, k, device="cuda"))[t]
        want = nf4_route.combine(y1, p1, torch.ones(1, k, device="cuda"))[0]
        assert torch.equal(got, want), f"token {t}"


@pytest.mark.parametrize("H,K,N_dn,rows", [(768, 2048, 2048, 4), (256, 4096, 512, 2),
                                           (320, 1024, 640, 2), (1024, 1536, 768, 3)])
def test_fused_ffn_gemv_forms_equal_the_composition(H, K, N_dn, rows):
    """Groups of 2..4 rows: gate_up GEMV with the silu epilogue, then the
    down stage in its own class (a GEMV at H = 320 and 1024 with 2..3 rows,
    the split-table kernels at H = 768 with 4 rows); and gate/up units of
    the single launch + down GEMV (K = 4096: only the down stage is a
    GEMV)."""
    import nf4_ffn
    from nf4_grouped import gemm_4bit_grouped
    E, G = 12, 20
    gu_p, gu_a = rand_nf4_stack(E, 2 * H, K, seed=H)
    dn_p, dn_a = rand_nf4_stack(E, N_dn, H, seed=H + 1)
    g = torch.Generator().manual_seed(H + rows)
    sizes = torch.randint(0, rows + 1, (G,), generator=g).tolist()
    sizes[3] = rows
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    a = rand_acts(sum(sizes), K, seed=12)
    fused = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
    gu = gemm_4bit_grouped(a, gu_p, gu_a, sizes, ids)
    comp = gemm_4bit_grouped(nf4_ffn.silu_mul_locked(gu), dn_p, dn_a, sizes, ids)
    assert torch.equal(fused, comp)
    for _ in range(3):
        again = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, ids, fused=True)
        assert torch.equal(again, comp)
    # every form leaves the sync words at zero (the gate/up-only single
    # launch has no down units, so its gate/up units set no flags)
    for (_d, _s), buf in nf4_ffn._SYNC.items():
        assert int(buf.abs().sum().item()) == 0
    assert not nf4_ffn.ffn_sync_error()
