"""Host logic of the device-side routing (no GPU): refusals, argument
checks, and the C ABI rejecting bad shapes before touching a device."""
import pytest
import torch

import _hiplib
import nf4_route


def test_cpu_tensors_are_refused():
    with pytest.raises(RuntimeError) as ei:
        nf4_route.route_topk(torch.zeros(2, 8), 2)
    assert "cuda" in str(ei.value).lower()
    with pytest.raises(RuntimeError):
        nf4_route.route_groups(torch.zeros(2, 2, dtype=torch.int64), 8)


def test_route_abi_rejects_bad_arguments_without_a_device():
    lib = _hiplib.load()
    topk = lib.gnf4_hip_route_topk
    assert topk(16, 4, 8, 8, 9, 0, 0, 16, 9, 16, 9, None) == -1     # k > E
    assert topk(16, 4, 8, 8, 65, 0, 0, 16, 65, 16, 65, None) == -1  # k > 64
    assert topk(16, 4, 2000, 2000, 8, 0, 0, 16, 8, 16, 8, None) == -1   # E > 1024
    assert topk(16, 4, 8, 8, 2, 2, 0, 16, 2, 16, 2, None) == -1     # mode
    assert topk(16, 4, 8, 4, 2, 0, 0, 16, 2, 16, 2, None) == -1     # ld < E
    assert topk(None, 0, 8, 8, 2, 0, 0, None, 2, None, 2, None) == 0   # nothing to do
    groups = lib.gnf4_hip_route_groups
    assert groups(16, 8, 2, 8, 600, 8, 0, 16, 16, 16, 16, 16, None) == -1  # E > 512
    assert groups(16, 4, 2, 8, 128, 8, 0, 16, 16, 16, 16, 16, None) == -1  # stride < k
    assert groups(16, 8, 2, 8, 128, 8, -1, 16, 16, 16, 16, 16, None) == -1  # cap < 0
    assert lib.gnf4_hip_gather_rows(16, 64, 16, 4, 2, 60, 16, 64, None) == -1     # K % 8
    assert lib.gnf4_hip_route_combine(16, 64, 16, 16, 1, 4, 2, 64, 16, 64, None) == -1
    routed = lib.gnf4_hip_grouped_decode_routed   # decode over routing tables
    assert routed(0, 16, 0, 64, 16, 32, 16, 16, 8, 2, 16, 16, 4, 0, 16, 64, 16, 16, None) == -1
    assert routed(0, 16, 0, 64, 16, 32, 16, 16, 8, 2, 16, None, 4, 2, 16, 64, 16, 16, None) == -1
    assert routed(0, 16, 0, 64, 16, 32, 16, 16, 8, 2, 16, 16, 0, 2, 16, 64, 16, 16, None) == 0


def test_plan_row_bound():
    plan = nf4_route.RoutePlan(*(torch.zeros(1),) * 5, T=3, k=8, E=128, slots=24)
    assert plan.rows == 24 and plan.max_rows_bound() == 3
    capped = nf4_route.RoutePlan(*(torch.zeros(1),) * 5, T=16, k=8, E=128, slots=128, cap=8)
    assert capped.max_rows_bound() == 8


def _groups_brute(N, E, cap, counts):
    return sum(0 if c == 0 else (-(-c // cap) if cap else 1) for c in counts)


def test_route_slots_hold_every_routing():
    """route_slots(N, E, cap) is at least the group count of every way N rows
    can fall on E experts (brute force over compositions for small N, E),
    and equals min(N, E) without a cap."""
    import itertools
    for N in range(1, 9):
        for E in range(1, 6):
            assert nf4_route.route_slots(N, E, 0) == min(N, E)
            for cap in (1, 2, 3, 8):
                worst = max(_groups_brute(N, E, cap, c)
                            for c in itertools.product(range(N + 1), repeat=E) if sum(c) == N)
                assert nf4_route.route_slots(N, E, cap) >= worst, (N, E, cap)
    # tight where it matters: 16 tokens x top-8 over 128 experts
    assert nf4_route.route_slots(128, 128, 8) == 128
    assert nf4_route.route_slots(128, 16, 8) == 16 + 112 // 8
