"""The no-allocation fused FFN entry point (gnf4_hip_nf4_ffn_fwd_noalloc)
against the allocating one (gnf4_hip_nf4_ffn_fwd), through the C ABI.

Both run the same kernel; only where the sync words live differs (a fixed
per-GPU array of the library vs a caller buffer), so the outputs must agree
bit for bit -- on two calls in a row, the second with a smaller input (the
array keeps the first call's contents), and when the same problem is run
again. Sizes beyond the array are rejected with -1 before any launch.
"""
import ctypes

import pytest
import torch

from _fixtures import rand_acts, rand_nf4_stack

pytestmark = pytest.mark.gpu


def _lib():
    import _hiplib
    return _hiplib.load()


def _problem(E, H, K, N_dn, sizes, ids, seed):
    gu_p, gu_a = rand_nf4_stack(E, 2 * H, K, seed)
    dn_p, dn_a = rand_nf4_stack(E, N_dn, H, seed + 1)
    a = rand_acts(sum(sizes), K, seed=seed + 2)
    row_off = [0]
    for m in sizes:
        row_off.append(row_off[-1] + m)
    dev = a.device
    eids = torch.tensor(ids, dtype=torch.int32, device=dev)
    ro = torch.tensor(row_off, dtype=torch.int32, device=dev)
    return a, gu_p, gu_a, dn_p, dn_a, eids, ro


def _args(a, gu_p, gu_a, dn_p, dn_a, eids, ro, G, max_m, h, out):
    T, K = a.shape
    H = gu_p.shape[1] // 2
    N_dn = dn_p.shape[1]
    head = (a.data_ptr(), 0, a.stride(0),
            gu_p.data_ptr(), gu_p.stride(0), gu_p.stride(1),
            gu_a.data_ptr(), gu_a.stride(0), gu_a.stride(1),
            dn_p.data_ptr(), dn_p.stride(0), dn_p.stride(1),
            dn_a.data_ptr(), dn_a.stride(0), dn_a.stride(1),
            eids.data_ptr(), ro.data_ptr(), G, max_m, 2 * H, K, N_dn,
            h.data_ptr(), h.stride(0))
    tail = (out.data_ptr(), out.stride(0), torch.cuda.current_stream().cuda_stream)
    return head, tail


def _run(noalloc, prob, sizes):
    lib = _lib()
    a, gu_p, gu_a, dn_p, dn_a, eids, ro = prob
    T = a.shape[0]
    H, N_dn = gu_p.shape[1] // 2, dn_p.shape[1]
    h = torch.empty(T, H, dtype=torch.bfloat16, device=a.device)
    out = torch.full((T, N_dn), 7.0, dtype=torch.bfloat16, device=a.device)
    head, tail = _args(*prob, len(sizes), max(sizes), h, out)
    if noalloc:
        rc = lib.gnf4_hip_nf4_ffn_fwd_noalloc(*head, *tail)
    else:
        words = int(lib.gnf4_hip_ffn_sync_words(len(sizes), 2 * H, N_dn))
        sync = torch.zeros(words, dtype=torch.int32, device=a.device)
        rc = lib.gnf4_hip_nf4_ffn_fwd(*head, sync.data_ptr(), words, *tail)
        torch.cuda.synchronize()
        assert int(sync[0].item()) == 0
        del sync
    assert rc == 0
    torch.cuda.synchronize()
    return out, h


def test_noalloc_matches_the_allocating_entry_point_on_two_calls():
    # first call: Qwen3-30B-A3B expert shape, batch-4 routing (groups of 1-2
    # rows, the split-codebook MFMA path); second: a smaller problem
    # (one-row groups, the fp32 FMA path) that reuses the array
    cases = [
        (128, 768, 2048, 2048, [2, 1, 1, 2, 1, 3, 1, 1, 2, 1, 1, 1, 1, 2, 1, 1, 2, 1, 1, 2,
                                1, 1, 1, 2, 1, 1], list(range(3, 120, 4))[:26], 80),
        (16, 256, 512, 384, [1, 1, 1], [9, 2, 14], 90),
    ]
    for E, H, K, N_dn, sizes, ids, seed in cases:
        prob = _problem(E, H, K, N_dn, sizes, ids, seed)
        want, want_h = _run(False, prob, sizes)
        got, got_h = _run(True, prob, sizes)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (E, H, K, N_dn)
        assert torch.equal(got_h.view(torch.int16), want_h.view(torch.int16))
        assert not torch.isnan(got.float()).any()
    # the first problem again after the smaller one
    E, H, K, N_dn, sizes, ids, seed = cases[0]
    prob = _problem(E, H, K, N_dn, sizes, ids, seed)
    want, _ = _run(False, prob, sizes)
    got, _ = _run(True, prob, sizes)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_rejects_sizes_beyond_its_array():
    lib = _lib()
    G, N_gu, N_dn = 128, 3072, 2048
    assert lib.gnf4_hip_ffn_sync_words(G, N_gu, N_dn) > (1 << 19)
    dummy = torch.zeros(64, dtype=torch.uint8, device="cuda")
    p = dummy.data_ptr()
    rc = lib.gnf4_hip_nf4_ffn_fwd_noalloc(p, 0, 2048, p, 16, 16, p, 16, 16, p, 16, 16, p, 16, 16,
                                          p, p, G, 1, N_gu, 2048, N_dn, p, 1536, p, 2048,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == -1


def _reset(lib):
    err = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    assert lib.gnf4_hip_nf4_ffn_noalloc_reset(err.data_ptr(),
                                              torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    return int(err.item())


def test_noalloc_reset_after_forced_time_outs_in_a_captured_graph():
    """A spin limit of 0 polls (forced from the host: a down unit that does
    not find its h ready at once gives up, and every kernel still exits) on
    a captured no-allocation call. Each replay's down units give either the
    allocating entry point's bits or NaN; the reset reports the error word
    exactly when some output is NaN and clears the array (flags the late
    gate/up units left included). A graph captured after it, with the normal
    limit, then replays exact, three times in a row."""
    lib = _lib()
    E, H, K, N_dn = 32, 512, 1024, 1024
    sizes, ids = [1, 3, 2, 4, 1, 1, 2, 2], [3, 7, 11, 15, 19, 23, 27, 31]
    prob = _problem(E, H, K, N_dn, sizes, ids, 95)
    want, _ = _run(False, prob, sizes)
    assert _reset(lib) == 0
    a = prob[0]
    T = a.shape[0]
    h = torch.empty(T, H, dtype=torch.bfloat16, device=a.device)
    out = torch.empty(T, N_dn, dtype=torch.bfloat16, device=a.device)

    def call():
        head, tail = _args(*prob, len(sizes), max(sizes), h, out)
        assert lib.gnf4_hip_nf4_ffn_fwd_noalloc(*head, *tail) == 0

    try:
        assert lib.gnf4_hip_ffn_set_spin_limit(0) == 0
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call()
    finally:
        assert lib.gnf4_hip_ffn_set_spin_limit(1 << 22) == 0
    for _ in range(3):
        out.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        nan = torch.isnan(out.float())
        row0 = 0
        for m in sizes:
            for c0 in range(0, N_dn, 32):
                blk = nan[row0:row0 + m, c0:c0 + 32]
                assert bool(blk.all()) or not bool(blk.any())
                if not bool(blk.any()):
                    assert torch.equal(out[row0:row0 + m, c0:c0 + 32].view(torch.int16),
                                       want[row0:row0 + m, c0:c0 + 32].view(torch.int16))
            row0 += m
        assert (_reset(lib) != 0) == bool(nan.any())
    assert _reset(lib) == 0
    del g
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        call()
    for _ in range(3):
        out.fill_(7.0)
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert _reset(lib) == 0
