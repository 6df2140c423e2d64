"""Write the golden vectors in this directory from the reference's own CPU
kernels (gnf4_native/cpu_kernels.c, compiled from its source into oracle/_ref
by oracle/Makefile). Run in a container that has the reference tree:

    make -C oracle && python tests/golden/make_golden.py

Each .npz holds the seeded inputs and the reference's fp32 outputs. The
fixture shapes and seeds follow the reference's own exactness tests
(kernel/test_cpu_grouped.py:16-54, :288-297, :339-363): E, N, K, G = 4, 24,
128, 3 with sizes [1, 2, 1] and ids [2, 0, 3]; MXFP4 scales 100..139 with
planted 0xFF / 0x00 bytes; dgrad K tails; groups larger than 8 rows; plus a
reduced config-1 slice (8 experts, K = 1024).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import native  # noqa: E402

E, N, K = 4, 24, 128
SIZES = [1, 2, 1]
EIDS = [2, 0, 3]


def nf4_stack(seed, rows, k=K, n=N):
    g = np.random.default_rng(seed)
    packed = g.integers(0, 256, size=(E, n, k // 2), dtype=np.uint8)
    absmax = g.random(size=(E, n, k // 64), dtype=np.float32) + 0.5
    a = g.standard_normal((rows, k), dtype=np.float32)
    return a, packed, absmax


def mx_stack(seed, rows, weird, k=K, n=N):
    g = np.random.default_rng(seed)
    packed = g.integers(0, 256, size=(E, n, k // 2), dtype=np.uint8)
    scales = g.integers(100, 140, size=(E, n, k // 32), dtype=np.uint8)
    if weird:
        scales[0, 0, 0] = 0xFF
        scales[0, 0, 1] = 0
        scales[1, 3, 2] = 0xFF
    a = g.standard_normal((rows, k), dtype=np.float32)
    return a, packed, scales


FFN_K, FFN_H, FFN_NDN = 128, 64, 24   # gu [E, 2H, K/2], dn [E, NDN, H/2]


def ffn_stack(seed, sizes, scale=1.0):
    """Fused-FFN inputs in the shape of the reference's own FFN tests
    (kernel/test_cpu_grouped.py:385-403); `scale` inflates the gu absmax so
    the gate values cross the silu clamps."""
    g = np.random.default_rng(seed)
    gu_p = g.integers(0, 256, size=(E, 2 * FFN_H, FFN_K // 2), dtype=np.uint8)
    gu_a = (g.random(size=(E, 2 * FFN_H, FFN_K // 64), dtype=np.float32) + 0.5) * np.float32(scale)
    dn_p = g.integers(0, 256, size=(E, FFN_NDN, FFN_H // 2), dtype=np.uint8)
    dn_a = g.random(size=(E, FFN_NDN, FFN_H // 64), dtype=np.float32) + 0.5
    a = g.standard_normal((sum(sizes), FFN_K), dtype=np.float32)
    eids = [int(x) for x in g.permutation(E)[:len(sizes)]]
    return a, gu_p, gu_a, dn_p, dn_a, list(sizes), eids


def ffn_cases():
    return {
        "ffn_nf4_groups_1_9_3": ffn_stack(21, (1, 9, 3)),
        "ffn_nf4_single_rows": ffn_stack(22, (1, 1, 1, 1)),
        "ffn_nf4_groups_8_8": ffn_stack(23, (8, 8)),
        "ffn_nf4_silu_clamps": ffn_stack(24, (2, 5), scale=40.0),
    }


def route_cases():
    """Router logits in the shape of the reference's epilogue test
    (kernel/test_cpu_grouped.py:158-188: t=3, e=64, k=8, a three-way tie),
    plus Qwen3 (E=128, top-8, renormalised) and GPT-OSS (E=32, top-4, softmax
    over the selection) shapes."""
    rng = np.random.default_rng(5)
    tie = rng.standard_normal((3, 64)).astype(np.float32)
    tie[0, 5] = tie[0, 11] = tie[0, 3]
    qwen = np.random.default_rng(6).standard_normal((16, 128)).astype(np.float32) * 2
    oss = np.random.default_rng(7).standard_normal((16, 32)).astype(np.float32) * 3
    return {
        "route_tie_mode0": (tie, 8, 0, 0), "route_tie_mode0_norm": (tie, 8, 0, 1),
        "route_tie_mode1": (tie, 8, 1, 0), "route_qwen3_top8_norm": (qwen, 8, 0, 1),
        "route_gptoss_top4": (oss, 4, 1, 0),
    }


def main():
    if native.ref_lib() is None:
        raise SystemExit("oracle/_ref is not built (needs the reference tree): make -C oracle")
    cases = {}
    a, p, s = nf4_stack(0, sum(SIZES))
    cases["gemv_nf4_fixture"] = ("gemv", "nf4", a, p, s, SIZES, EIDS)
    a, p, s = mx_stack(1, sum(SIZES), weird=True)
    cases["gemv_mxfp4_weird_scales"] = ("gemv", "mxfp4", a, p, s, SIZES, EIDS)
    for sizes in ([9], [16], [8, 17, 1], [33, 2]):
        eids = [i % E for i in range(len(sizes))]
        a, p, s = nf4_stack(0, sum(sizes))
        cases["gemv_nf4_groups_" + "_".join(map(str, sizes))] = ("gemv", "nf4", a, p, s, sizes, eids)
        a, p, s = mx_stack(1, sum(sizes), weird=False)
        cases["gemv_mxfp4_groups_" + "_".join(map(str, sizes))] = ("gemv", "mxfp4", a, p, s, sizes, eids)
    g, p, s = nf4_stack(5, sum(SIZES))
    g = np.random.default_rng(55).standard_normal((sum(SIZES), N), dtype=np.float32)
    cases["dgrad_nf4_fixture"] = ("dgrad", "nf4", g, p, s, SIZES, EIDS)
    for k in (64, 192, 320):
        _, p, s = nf4_stack(17, 1, k=k)
        g = np.random.default_rng(170 + k).standard_normal((sum(SIZES), N), dtype=np.float32)
        cases[f"dgrad_nf4_k{k}"] = ("dgrad", "nf4", g, p, s, SIZES, EIDS)
    _, p, s = mx_stack(7, 1, weird=True)
    s[2, 5, 2] = 0xFF
    g = np.random.default_rng(77).standard_normal((sum(SIZES), N), dtype=np.float32)
    cases["dgrad_mxfp4_weird_scales"] = ("dgrad", "mxfp4", g, p, s, SIZES, EIDS)
    sizes = [12, 1, 20]
    _, p, s = nf4_stack(13, 1)
    g = np.random.default_rng(131).standard_normal((sum(sizes), N), dtype=np.float32)
    cases["dgrad_nf4_training_groups"] = ("dgrad", "nf4", g, p, s, sizes, [1, 3, 0])
    # config-1 slice: 8 experts, N = 64 rows each, K = 1024, 4 rows per expert
    rng = np.random.default_rng(2024)
    p8 = rng.integers(0, 256, size=(8, 64, 512), dtype=np.uint8)
    s8 = (rng.random(size=(8, 64, 16), dtype=np.float32) * 0.05 + 0.01).astype(np.float32)
    a8 = rng.standard_normal((32, 1024), dtype=np.float32)
    cases["gemv_nf4_config1_slice"] = ("gemv", "nf4", a8, p8, s8, [4] * 8, list(range(8)))

    only = sys.argv[1] if len(sys.argv) > 1 else ""
    for name, (lg, k, mode, norm) in route_cases().items():
        if name.startswith(only):
            idx, wts = native.ref_route_topk(lg, k, mode, norm)
            np.savez_compressed(HERE / f"{name}.npz", op="route", logits=lg, k=k, mode=mode,
                                norm=norm, idx=idx, wts=wts,
                                ref_build=str(native.ref_path().name))
            print(name, idx.shape)
    for name, args in ffn_cases().items():
        if name.startswith(only):
            x, gu_p, gu_a, dn_p, dn_a, sizes, eids = args
            out = native.ref_ffn_grouped(x, gu_p, gu_a, dn_p, dn_a, sizes, eids, threads=1)
            np.savez_compressed(HERE / f"{name}.npz", op="ffn", fmt="nf4", x=x, gu_packed=gu_p,
                                gu_absmax=gu_a, dn_packed=dn_p, dn_absmax=dn_a,
                                sizes=np.asarray(sizes, np.int32),
                                eids=np.asarray(eids, np.int64), out=out,
                                ref_build=str(native.ref_path().name))
            print(name, out.shape)
    for name, (op, fmt, x, p, s, sizes, eids) in cases.items():
        if not name.startswith(only):
            continue
        fn = native.ref_gemv_grouped if op == "gemv" else native.ref_dgrad_grouped
        out = fn(x, p, s, sizes, eids, fmt=fmt, threads=1)
        np.savez_compressed(HERE / f"{name}.npz", op=op, fmt=fmt, x=x, packed=p, scales=s,
                            sizes=np.asarray(sizes, np.int32), eids=np.asarray(eids, np.int64),
                            out=out, ref_build=str(native.ref_path().name))
        print(name, out.shape)


if __name__ == "__main__":
    main()
