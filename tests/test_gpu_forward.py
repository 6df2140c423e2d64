"""GPU parity of the forward ops against the oracle and the tolerance contract.

Bars (reference docs/TOLERANCE_CONTRACT.md, kernel/test_nf4_grouped.py):
  * decode/unpack: bit-exact. One-hot activations make each output a single
    decoded weight, so out == dequant(W).to(bf16) exactly, for every code in
    both nibble positions, on both kernels (decode and tiled).
  * full outputs: B-abs rel-Frobenius <= 1e-2 vs fp64 and B-rel <= 2x the bf16
    dequant-then-matmul path; agreement with the C oracle (the reference's
    locked CPU tree) within 1e-2 relative.
"""
import numpy as np
import pytest
import torch

from _fixtures import (contract_check, dequant, oracle_fwd, rand_acts, rand_mx_stack,
                       rand_nf4_stack, rel_err, spread_ids)

pytestmark = pytest.mark.gpu


def _ops():
    from mxfp4_grouped import gemm_mxfp4_grouped
    from nf4_grouped import gemm_4bit_grouped
    return {"nf4": gemm_4bit_grouped, "mxfp4": gemm_mxfp4_grouped}


def _stack(fmt, E, N, K, seed=0):
    return rand_nf4_stack(E, N, K, seed) if fmt == "nf4" else rand_mx_stack(E, N, K, seed)


def test_native_library_is_the_one_in_tree():
    import _hiplib
    lib = _hiplib.load()
    assert lib.gnf4_hip_abi_version() == _hiplib.ABI_VERSION
    assert lib.gnf4_hip_device_cus() > 0
    assert str(_hiplib.LIB_PATH).endswith("grouped-nf4-gemm_amd/libgnf4_hip.so")


# ------------------------------------------------------------ exactness --

@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_all_codes_both_nibble_positions_tiled(fmt):
    """Every (code, position) pair via one-hot rows (reference
    kernel/test_nf4_grouped.py:92-109): K one-hot rows -> tiled kernel."""
    N, K = 16, 64
    B = torch.empty(1, N, K // 2, dtype=torch.uint8, device="cuda")
    for c in range(16):
        B[0, c, :] = (c << 4) | (15 - c)
    if fmt == "nf4":
        S = torch.ones(1, N, K // 64, dtype=torch.float32, device="cuda")
    else:
        S = torch.full((1, N, K // 32), 127, dtype=torch.uint8, device="cuda")
    eye = torch.eye(K, dtype=torch.bfloat16, device="cuda")
    out = _ops()[fmt](eye, B, S, [K], [0])
    ref = dequant(fmt, B[0], S[0])
    assert torch.equal(out.t(), ref.to(torch.bfloat16))


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_every_byte_every_position_with_scales(fmt):
    """All 256 byte values in every row, random per-block scales: the one-hot
    product through the tiled kernel equals the bf16-rounded decode."""
    N, K = 48, 512
    g = torch.Generator().manual_seed(5)
    perm = torch.stack([torch.randperm(256, generator=g) for _ in range(N)]).to(torch.uint8)
    B = perm.reshape(1, N, 256).cuda()
    if fmt == "nf4":
        S = (torch.rand(1, N, K // 64, generator=g) * 4 + 0.01).cuda()
    else:
        S = torch.randint(100, 150, (1, N, K // 32), generator=g, dtype=torch.uint8).cuda()
    eye = torch.eye(K, dtype=torch.bfloat16, device="cuda")
    out = _ops()[fmt](eye, B, S, [K], [0])
    ref = dequant(fmt, B[0], S[0]).to(torch.bfloat16)
    assert torch.equal(out.t(), ref)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("k_hot", [0, 100, 511])
def test_decode_kernel_one_hot_exact(fmt, k_hot):
    """Decode kernel (M = 1): a one-hot row selects one weight column exactly
    (reference kernel/test_nf4_grouped.py:257-265)."""
    N, K = 144, 512
    B, S = _stack(fmt, 3, N, K, seed=7)
    a = torch.zeros(1, K, dtype=torch.bfloat16, device="cuda")
    a[0, k_hot] = 1.0
    out = _ops()[fmt](a, B, S, [1], [2])
    ref = dequant(fmt, B[2], S[2])[:, k_hot].to(torch.bfloat16)
    assert torch.equal(out[0], ref)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_decode_kernel_sixteen_one_hot_rows(fmt):
    """A 16-row group through the decode kernel: row r one-hot at k = 37 r."""
    N, K = 64, 640
    B, S = _stack(fmt, 2, N, K, seed=9)
    a = torch.zeros(16, K, dtype=torch.bfloat16, device="cuda")
    for r in range(16):
        a[r, 37 * r] = 1.0
    out = _ops()[fmt](a, B, S, [16], [1])
    w = dequant(fmt, B[1], S[1]).to(torch.bfloat16)
    for r in range(16):
        assert torch.equal(out[r], w[:, 37 * r]), r


# ------------------------------------------------------------- tolerance --

SHAPES = [  # (name, fmt, N, K, E, k)
    ("c1_tiny", "nf4", 512, 1024, 8, 8),
    ("qwen_gu", "nf4", 1536, 2048, 128, 8),
    ("qwen_dn", "nf4", 2048, 768, 128, 8),
    ("gptoss_gu", "mxfp4", 5760, 2880, 32, 4),
    ("gptoss_dn", "mxfp4", 2880, 2880, 32, 4),
]


def _census_case(name, fmt, N, K, E, k, m):
    active = spread_ids(E, k)
    Wa, Sa = _stack(fmt, len(active), N, K, seed=11)
    # a stack of E experts where only the active ids are populated
    W = torch.zeros(E, N, K // 2, dtype=torch.uint8, device="cuda")
    S = torch.zeros((E, N, K // (64 if fmt == "nf4" else 32)), dtype=Sa.dtype, device="cuda")
    W[active] = Wa
    S[active] = Sa
    sizes = [m] * len(active)
    a = rand_acts(sum(sizes), K, seed=12)
    out = _ops()[fmt](a, W, S, sizes, active)
    return contract_check(fmt, out, a, W, S, sizes, active)


@pytest.mark.parametrize("name,fmt,N,K,E,k", SHAPES)
@pytest.mark.parametrize("m", [1, 4, 16, 128, 290])
def test_contract_census_shapes(name, fmt, N, K, E, k, m):
    """B-abs and B-rel on every census shape and regime, and the fidelity
    ordering P-fid (reference docs/TOLERANCE_CONTRACT.md:16-25) per regime:
      * NF4 decode (groups of <= 16 rows): the kernels sum fp32 codebook
        values (exact three-part bf16 split, or fp32 FMAs for one-row
        groups) and scale by absmax once per block in fp32, so their error
        must be strictly below the bf16 dequant path's;
      * NF4 tiles (> 16 rows): bf16 weights bf16(codebook * absmax) into bf16
        MFMA, the reference's opt-in VARIANT 3 (kernel/nf4_grouped.py:438-445,
        "P-fid parity"): the errors tie, within 1 %;
      * MXFP4: e2m1 * 2^e is exact in bf16, so both paths hold the same
        weights and the errors tie, within 1 %."""
    e_f, e_d = _census_case(name, fmt, N, K, E, k, m)
    print(f"PFID {name} m={m}: fused {e_f:.3e} dequant {e_d:.3e} ratio {e_f / e_d:.4f}")
    if fmt == "nf4" and m <= 16:
        assert e_f <= 0.9 * e_d, f"P-fid (decode): {e_f:.3e} vs dequant {e_d:.3e}"
    else:
        assert e_f <= 1.01 * e_d, f"P-fid (parity): {e_f:.3e} vs dequant {e_d:.3e}"


def test_pfid_median_over_the_nf4_census():
    """P-fid as the contract registers it: the median over the census shapes
    and regimes (decode batch 1 / 4 / 16 rows per expert, prefill 128 / 290)
    of fused error / dequant-path error is at most 1."""
    ratios = []
    for name, fmt, N, K, E, k in SHAPES:
        if fmt != "nf4":
            continue
        for m in (1, 4, 16, 128, 290):
            e_f, e_d = _census_case(name, fmt, N, K, E, k, m)
            ratios.append(e_f / e_d)
    med = float(np.median(ratios))
    print(f"PFID median over {len(ratios)} NF4 census cases: {med:.4f}")
    assert med <= 1.0, ratios


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("sizes,ids", [([1] * 8, list(range(8))),
                                       ([4, 1, 2, 3], [7, 0, 3, 5]),
                                       ([33, 2, 70], [1, 6, 4])])
def test_agrees_with_the_c_oracle(fmt, sizes, ids):
    """The GPU output against the reference's locked CPU tree (restated in
    oracle/gnf4_oracle.c, bit-exact to the compiled reference)."""
    N, K = 512, 1024
    W, S = _stack(fmt, 8, N, K, seed=3)
    a = rand_acts(sum(sizes), K, seed=4)
    out = _ops()[fmt](a, W, S, sizes, ids)
    ref = torch.from_numpy(oracle_fwd(fmt, a, W, S, sizes, ids))
    assert rel_err(out.float().cpu(), ref) < 1e-2


# ------------------------------------------------------------ boundaries --

@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_single_token_groups(fmt):
    W, S = _stack(fmt, 8, 128, 128)
    a = rand_acts(3, 128)
    out = _ops()[fmt](a, W, S, [1, 1, 1], [2, 5, 7])
    assert out.shape == (3, 128)
    contract_check(fmt, out, a, W, S, [1, 1, 1], [2, 5, 7])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_all_tokens_one_expert(fmt):
    W, S = _stack(fmt, 8, 128, 128)
    a = rand_acts(200, 128)
    out = _ops()[fmt](a, W, S, [200], [3])
    contract_check(fmt, out, a, W, S, [200], [3])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_noncontiguous_unsorted_ids(fmt):
    W, S = _stack(fmt, 8, 128, 128)
    a = rand_acts(30, 128)
    sizes, ids = [10, 5, 15], [6, 1, 4]
    out = _ops()[fmt](a, W, S, sizes, ids)
    contract_check(fmt, out, a, W, S, sizes, ids)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("m", [1, 5, 40])
def test_k_equals_blocksize(fmt, m):
    K = 64 if fmt == "nf4" else 32
    W, S = _stack(fmt, 2, 64, K)
    a = rand_acts(m, K)
    out = _ops()[fmt](a, W, S, [m], [1])
    contract_check(fmt, out, a, W, S, [m], [1])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_ragged_tail_tiles_and_n_tail(fmt):
    W, S = _stack(fmt, 8, 200, 192)
    a = rand_acts(65 + 17, 192)
    out = _ops()[fmt](a, W, S, [65, 17], [0, 7], block_m=64)
    contract_check(fmt, out, a, W, S, [65, 17], [0, 7])


@pytest.mark.parametrize("K", [32, 96, 160, 2880])
def test_mxfp4_k_not_a_multiple_of_64(K):
    W, S = rand_mx_stack(3, 96, K)
    for sizes in ([1, 1], [3, 9], [20, 50]):
        a = rand_acts(sum(sizes), K)
        out = _ops()["mxfp4"](a, W, S, sizes, [2, 0])
        contract_check("mxfp4", out, a, W, S, sizes, [2, 0])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_expert_id_forms_bitwise_equal_with_empty_group(fmt):
    """list / CPU tensor / device tensor ids give identical bits, including a
    zero-size group (reference kernel/test_eids_forms.py:27, :66-92)."""
    W, S = _stack(fmt, 6, 256, 256)
    sizes = [3, 1, 0, 5, 2]
    ids = [4, 0, 2, 5, 1]
    a = rand_acts(sum(sizes), 256)
    op = _ops()[fmt]
    for bm in (None, 16):
        base = op(a, W, S, sizes, ids, block_m=bm)
        cpu_t = op(a, W, S, sizes, torch.tensor(ids, dtype=torch.int32), block_m=bm)
        dev_t = op(a, W, S, sizes, torch.tensor(ids, dtype=torch.int64, device="cuda"), block_m=bm)
        assert torch.equal(base, cpu_t) and torch.equal(base, dev_t)
        keep = [i for i, m in enumerate(sizes) if m]
        contract_check(fmt, base, a, W, S, [sizes[i] for i in keep], [ids[i] for i in keep])


def test_sizes_tensor_is_not_mutated():
    from nf4_grouped import gemm_4bit_grouped
    W, S = rand_nf4_stack(4, 128, 128)
    sizes = torch.tensor([40, 0, 25])
    a = rand_acts(65, 128)
    gemm_4bit_grouped(a, W, S, sizes, [0, 1, 2])
    out2 = gemm_4bit_grouped(a, W, S, sizes, [0, 1, 2])
    assert sizes.tolist() == [40, 0, 25]
    assert out2.shape == (65, 128)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_repeat_runs_bitwise_identical(fmt):
    """Determinism: same inputs, same bits (no atomics in any reduction)."""
    W, S = _stack(fmt, 16, 768, 1024)
    for sizes in ([1] * 12, [3, 16, 2, 9], [130, 7, 64]):
        ids = list(range(len(sizes)))
        a = rand_acts(sum(sizes), 1024)
        x = _ops()[fmt](a, W, S, sizes, ids)
        y = _ops()[fmt](a, W, S, sizes, ids)
        assert torch.equal(x, y)


def test_split_k_and_tuning_knobs_keep_the_result():
    """The reference's schedule knobs are accepted and leave the bits alone."""
    from nf4_grouped import gemm_4bit_grouped
    W, S = rand_nf4_stack(8, 512, 2048)
    a = rand_acts(2, 2048)
    one = gemm_4bit_grouped(a, W, S, [1, 1], [0, 4], split_k=1)
    for sk in (2, 4, 8):
        assert torch.equal(gemm_4bit_grouped(a, W, S, [1, 1], [0, 4], split_k=sk), one)
    assert torch.equal(gemm_4bit_grouped(a, W, S, [1, 1], [0, 4], decode_config=(128, 4)), one)
    a2 = rand_acts(256, 2048)
    base = gemm_4bit_grouped(a2, W, S, [128, 128], [1, 5])
    for kw in (dict(prefill_config=(64, 4, 3)), dict(prefill_variant=0),
               dict(prefill_variant=3), dict(prefill_groups=2)):
        assert torch.equal(gemm_4bit_grouped(a2, W, S, [128, 128], [1, 5], **kw), base)
    with pytest.raises(ValueError, match="prefill_variant"):
        gemm_4bit_grouped(a2, W, S, [128, 128], [1, 5], prefill_variant=2)


def test_stack_beyond_2gib_offsets():
    """Experts on both sides of a 2^31-byte stack (reference
    kernel/test_offsets_2gib.py:79-110): 64-bit offset arithmetic."""
    from nf4_grouped import gemm_4bit_grouped
    E, N, K = 257, 4096, 4096          # 8 MiB per expert -> 2.01 GiB stack
    W = torch.randint(0, 256, (E, N, K // 2), dtype=torch.uint8, device="cuda")
    S = torch.rand(E, N, K // 64, device="cuda") * 0.05 + 0.01
    assert W.numel() > 2 ** 31
    ids = [0, 128, 256]
    for m in (1, 40):
        a = rand_acts(3 * m, K)
        out = gemm_4bit_grouped(a, W, S, [m] * 3, ids)
        contract_check("nf4", out, a, W, S, [m] * 3, ids)
    del W


def test_mxfp4_e8m0_edges_follow_exp2_multiply():
    """0xFF decodes as 2^128 (inf for nonzero codes, NaN for zero codes);
    0x00 as 2^-127: the decoded weights are bf16 subnormals, which the
    conversion and the MFMA keep. The one-hot path shows the decoded value
    directly."""
    from mxfp4_grouped import gemm_mxfp4_grouped
    N, K = 16, 64
    B = torch.empty(1, N, K // 2, dtype=torch.uint8, device="cuda")
    B[0, :, :] = 0x21                    # elements (0.5, 1.0) pairwise
    S = torch.full((1, N, K // 32), 127, dtype=torch.uint8, device="cuda")
    S[0, 1, :] = 0                        # subnormal scale 2^-127
    S[0, 2, :] = 130
    a = torch.zeros(1, K, dtype=torch.bfloat16, device="cuda")
    a[0, 1] = 1.0                         # element 1 = high nibble of byte 0 = 1.0
    out = gemm_mxfp4_grouped(a, B, S, [1], [0]).float()
    assert out[0, 0].item() == 1.0
    assert out[0, 2].item() == 8.0
    assert out[0, 1].item() == 2.0 ** -127           # subnormal kept


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("rows", [1, 5, 40, 300])
def test_subnormal_decoded_weights_are_kept(fmt, rows):
    """Scales that make every decoded weight subnormal (MXFP4 e8m0 0x00, so
    2^-127 * e2m1; NF4 absmax 1e-38) through the decode (1 and 5 rows) and
    tiled (40 and 300 rows) kernels: one-hot rows reproduce the decoded
    weights bit for bit, subnormals included."""
    N, K = 64, 256
    g = torch.Generator().manual_seed(21)
    B = torch.randint(0, 256, (1, N, K // 2), generator=g, dtype=torch.uint8).cuda()
    if fmt == "nf4":
        S = torch.full((1, N, K // 64), 1e-38, dtype=torch.float32, device="cuda")
    else:
        S = torch.zeros((1, N, K // 32), dtype=torch.uint8, device="cuda")
    k = torch.arange(rows, device="cuda") * 7 % K
    a = torch.zeros(rows, K, dtype=torch.bfloat16, device="cuda")
    a[torch.arange(rows, device="cuda"), k] = 1.0
    out = _ops()[fmt](a, B, S, [rows], [0])
    want = dequant(fmt, B[0], S[0]).to(torch.bfloat16).t()[k]
    assert bool((want != 0).any())
    assert torch.equal(out, want)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_planned_launch_matches_the_op_and_replays_in_a_graph(fmt):
    """GroupPlan + launch_planned (device-resident group tables) give the op's
    bits, also when captured in a graph and replayed with eager work between."""
    from nf4_grouped import GroupPlan, launch_planned
    code = 0 if fmt == "nf4" else 1
    W, S = _stack(fmt, 16, 512, 1024)
    dev = torch.device("cuda:0")
    for sizes, ids in (([1] * 8, list(range(8))), ([3, 0, 16, 2], [5, 1, 9, 0]),
                       ([40, 130, 1], [2, 7, 3])):
        a = rand_acts(sum(sizes), 1024)
        ref = _ops()[fmt](a, W, S, sizes, ids)
        plan = GroupPlan(sizes, ids, dev)
        assert torch.equal(launch_planned(code, a, W, S, plan), ref)
        out = torch.empty_like(ref)
        launch_planned(code, a, W, S, plan, out=out)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            launch_planned(code, a, W, S, plan, out=out)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            launch_planned(code, a, W, S, plan, out=out)
        for _ in range(3):
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("sizes", [[300, 17, 129, 256, 1, 600], [257], [128, 130]])
def test_tall_tiles_give_the_bits_of_128_row_tiles(fmt, sizes):
    """256-row tiles (the default above 128 rows) change how rows are
    batched, never an output's arithmetic: bitwise equal to 128-row tiles,
    tail tiles of <= 128 rows included."""
    N, K = 512, 1024
    W, S = _stack(fmt, 8, N, K, seed=61)
    ids = list(range(len(sizes)))
    a = rand_acts(sum(sizes), K, seed=62)
    op = _ops()[fmt]
    tall = op(a, W, S, sizes, ids, block_m=256)
    short = op(a, W, S, sizes, ids, block_m=128)
    auto = op(a, W, S, sizes, ids)
    assert torch.equal(tall, short) and torch.equal(auto, tall)
    contract_check(fmt, tall, a, W, S, sizes, ids)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("N,K", [(320, 704), (2880, 2880), (96, 64), (260, 256), (1540, 384)])
def test_tall_tiles_ragged_weight_rows_and_step_counts(fmt, N, K):
    """The four-wave tall-tile kernel with weight rows that do not fill its
    256-row tile (N % 256 != 0), step counts that are not multiples of the
    three-slot load rings (K / 64 = 11, 45, 1), output widths that end
    inside an 8-column store chunk (N % 8 == 4) and every row-subtile class
    (<= 64, <= 128, > 128 rows): bitwise equal to 128-row tiles."""
    sizes = [300, 40, 0, 100, 256, 129]
    W, S = _stack(fmt, 6, N, K, seed=71)
    ids = [5, 0, 3, 1, 2, 4]
    a = rand_acts(sum(sizes), K, seed=72)
    op = _ops()[fmt]
    tall = op(a, W, S, sizes, ids, block_m=256)
    short = op(a, W, S, sizes, ids, block_m=128)
    assert torch.equal(tall, short)
    contract_check(fmt, tall, a, W, S, sizes, ids)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_decode_more_than_65535_one_row_groups(fmt):
    """One-row groups beyond the grid's 65535 rows run as several launches
    over consecutive group ranges: every row equals the same row computed in
    a smaller call, bit for bit, and the whole meets the contract."""
    E, N, K, T = 4, 32, 128, 70000
    W, S = _stack(fmt, E, N, K, seed=21)
    a = rand_acts(T, K, seed=22)
    ids = torch.randint(0, E, (T,), generator=torch.Generator().manual_seed(23)).tolist()
    op = _ops()[fmt]
    out = op(a, W, S, [1] * T, ids)
    head = op(a[:40000], W, S, [1] * 40000, ids[:40000])
    tail = op(a[40000:], W, S, [1] * (T - 40000), ids[40000:])
    assert torch.equal(out, torch.cat([head, tail]))
    sel = list(range(0, T, 997))
    contract_check(fmt, out[sel], a[sel], W, S, [1] * len(sel), [ids[i] for i in sel])


@pytest.mark.parametrize("fmt,N,K", [("nf4", 1536, 2048), ("nf4", 2048, 768), ("mxfp4", 2880, 2880),
                                     ("mxfp4", 640, 1440)])
def test_decode_group_rows_do_not_depend_on_the_batch(fmt, N, K):
    """A group's decoded rows are the same bits in a launch of many units as
    in a launch of that group with only the batch's largest group beside it,
    and the whole meets the contract. The largest group fixes the launch's
    class (NF4: one row, up to 8 rows, 9..16 rows; MXFP4: one row, more
    rows: the arithmetic and the chunks per wave differ between classes);
    within a class no group's bits depend on the others. Covers ragged groups, empty groups, a K tail
    (2880 = 22.5 chunks) and N past a 128-row boundary."""
    E = 24
    W, S = _stack(fmt, E, N, K, seed=31)
    g = torch.Generator().manual_seed(32)
    G = 120 if N >= 1536 else 400
    sizes = torch.randint(0, 17, (G,), generator=g).tolist()
    sizes[3] = 0
    sizes[5] = 16
    sizes[7] = 1
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    a = rand_acts(sum(sizes), K, seed=33)
    op = _ops()[fmt]
    out = op(a, W, S, sizes, ids)
    r5 = sum(sizes[:5])
    for gi in (0, 1, 7, G - 1):
        r0 = sum(sizes[:gi])
        m = sizes[gi]
        if m == 0:
            continue
        pair = op(torch.cat([a[r0:r0 + m], a[r5:r5 + 16]]), W, S, [m, 16], [ids[gi], ids[5]])
        assert torch.equal(out[r0:r0 + m], pair[:m]), f"group {gi} differs"
    sel = list(range(0, sum(sizes), 7))
    contract_check(fmt, out[sel], a[sel], W, S, [1] * len(sel),
                   [ids[next(i for i in range(G) if sum(sizes[:i + 1]) > r)] for r in sel])


@pytest.mark.parametrize("fmt,N,K,rows,G", [("nf4", 1536, 2048, 8, 60), ("nf4", 648, 1536, 5, 60),
                                            ("nf4", 1536, 2048, 3, 86), ("nf4", 640, 1024, 5, 60),
                                            ("mxfp4", 5760, 2880, 16, 60),
                                            ("mxfp4", 2880, 2880, 9, 60),
                                            ("mxfp4", 1560, 2880, 3, 60),
                                            ("mxfp4", 1560, 2880, 4, 20)])
def test_streamed_decode_matches_the_per_unit_kernel(fmt, N, K, rows, G):
    """Batched launches (20..86 groups) run the unit walks -- MXFP4 at
    K = 2880 (2..16 rows; 20 groups: walks of 5 units), NF4 at
    1024 < K <= 2048 (2..8 rows); a launch of
    one or two groups runs the per-unit kernel. Both must give the same bits
    for every group (NF4: all of them; same chunk split per wave, same
    reduction order), with
    ragged groups, an empty group, a partial last unit (N = 1560, 648) and a
    K tail (MXFP4 22.5 chunks). K = 1024 (one chunk per wave) stays on the
    per-unit kernel: the invariance holds there too."""
    E = 40
    W, S = _stack(fmt, E, N, K, seed=41)
    g = torch.Generator().manual_seed(42)
    sizes = torch.randint(1, rows + 1, (G,), generator=g).tolist()
    sizes[2] = 0
    sizes[4] = rows
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    a = rand_acts(sum(sizes), K, seed=43)
    op = _ops()[fmt]
    out = op(a, W, S, sizes, ids)
    for gi in (range(G) if fmt == "nf4" else (0, 1, 4, 17, G - 1)):
        r0, m = sum(sizes[:gi]), sizes[gi]
        if m == 0:
            continue
        # one group alone, beside a group of the batch's largest size, which
        # keeps the launch class (a launch of one-row groups takes the
        # one-row GEMV, in either format); two groups still take the
        # per-unit kernel at these shapes
        pad = rows if m < rows else 0
        aa = torch.cat([a[r0:r0 + m], a[:pad]]) if pad else a[r0:r0 + m]
        alone = op(aa, W, S, [m] + ([pad] if pad else []), [ids[gi]] + ([ids[gi]] if pad else []))
        assert torch.equal(out[r0:r0 + m], alone[:m]), f"group {gi} differs"
    sel = list(range(0, sum(sizes), 5))
    contract_check(fmt, out[sel], a[sel], W, S, [1] * len(sel),
                   [ids[next(i for i in range(G) if sum(sizes[:i + 1]) > r)] for r in sel])


def test_streamed_mxfp4_scales_off_16_byte_alignment():
    """The MXFP4 unit walk moves each unit's scale bytes through LDS with
    16-byte loads when the scale stack is 16-byte aligned, and loads them per
    lane otherwise. Scales one byte off alignment take the per-lane form:
    the same bits as the aligned stack, and as the per-unit kernel."""
    N, K, rows, G, E = 1560, 2880, 3, 60, 40
    W, S = _stack("mxfp4", E, N, K, seed=51)
    buf = torch.empty(S.numel() + 1, dtype=torch.uint8, device=S.device)
    S1 = buf[1:].view(S.shape)
    S1.copy_(S)
    assert S1.data_ptr() % 16 != 0
    g = torch.Generator().manual_seed(52)
    sizes = torch.randint(1, rows + 1, (G,), generator=g).tolist()
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    a = rand_acts(sum(sizes), K, seed=53)
    op = _ops()["mxfp4"]
    out = op(a, W, S, sizes, ids)
    assert torch.equal(op(a, W, S1, sizes, ids), out)
    for gi in (0, 7, G - 1):
        r0, m = sum(sizes[:gi]), sizes[gi]
        assert torch.equal(out[r0:r0 + m], op(a[r0:r0 + m], W, S1, [m], [ids[gi]])), gi


def test_row_stream_nf4_absmax_off_16_byte_alignment():
    """The NF4 row-streaming decode (K = 768, groups of 2..8 rows) reads a
    tile's absmax as one coalesced 16-row block when the absmax stack is
    16-byte aligned, and per chunk pair otherwise: an absmax stack one float
    off alignment gives the same bits."""
    N, K, G, E = 2048, 768, 40, 16
    W, S = _stack("nf4", E, N, K, seed=61)
    buf = torch.empty(S.numel() + 1, dtype=S.dtype, device=S.device)
    S1 = buf[1:].view(S.shape)
    S1.copy_(S)
    assert S1.data_ptr() % 16 != 0
    g = torch.Generator().manual_seed(62)
    sizes = torch.randint(2, 9, (G,), generator=g).tolist()
    ids = torch.randint(0, E, (G,), generator=g).tolist()
    a = rand_acts(sum(sizes), K, seed=63)
    op = _ops()["nf4"]
    out = op(a, W, S, sizes, ids)
    assert torch.equal(op(a, W, S1, sizes, ids), out)
    sel = list(range(0, sum(sizes), 3))
    contract_check("nf4", out[sel], a[sel], W, S, [1] * len(sel),
                   [ids[next(i for i in range(G) if sum(sizes[:i + 1]) > r)] for r in sel])


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_tall_tiles_several_per_workgroup(fmt):
    """More 256-row tiles than the persistent grid has workgroups (64 groups
    of mixed heights x 8 weight-row tiles), so each workgroup runs several
    tiles of different row-subtile classes back to back, reusing its LDS and
    pair table: bitwise equal to 128-row tiles and inside the contract."""
    N, K, E = 2048, 256, 64
    rng = np.random.default_rng(81)
    sizes = [int(v) for v in rng.choice([300, 256, 200, 129, 128, 100, 65, 64, 40, 1], size=E)]
    W, S = _stack(fmt, E, N, K, seed=82)
    ids = [int(v) for v in rng.permutation(E)]
    a = rand_acts(sum(sizes), K, seed=83)
    op = _ops()[fmt]
    tall = op(a, W, S, sizes, ids, block_m=256)
    short = op(a, W, S, sizes, ids, block_m=128)
    assert torch.equal(tall, short)
    contract_check(fmt, tall, a, W, S, sizes, ids)


def test_group_table_ring_wraps_without_reuse_races():
    """Eager calls stage their group tables in a pinned ring (eight parts,
    event-guarded): decode launches read them there at the ring's device
    address, tile launches from a device copy. 1200 back-to-back calls
    cycling two decode routings and one tiled routing wrap the ring more
    than twice; every output must equal its routing's result computed from
    device-resident expert ids (no ring) bit for bit, with no host sync
    between the launches."""
    import nf4_grouped
    from nf4_grouped import gemm_4bit_grouped
    W, S = _stack("nf4", 32, 256, 512, seed=91)
    g = torch.Generator().manual_seed(92)
    routes = []
    for lo, hi, G in ((1, 4, 64), (1, 4, 64), (150, 300, 6)):
        sizes = torch.randint(lo, hi, (G,), generator=g).tolist()
        ids = torch.randint(0, 32, (G,), generator=g).tolist()
        routes.append((sizes, ids, rand_acts(sum(sizes), 512, seed=93 + G)))
    refs = [gemm_4bit_grouped(a, W, S, sizes, torch.tensor(ids, dtype=torch.int32, device="cuda"))
            for sizes, ids, a in routes]
    outs = []
    for i in range(1200):
        sizes, ids, a = routes[i % 3]
        outs.append(gemm_4bit_grouped(a, W, S, sizes, ids))
    torch.cuda.synchronize()
    ring = nf4_grouped._table_ring(torch.device("cuda", torch.cuda.current_device()),
                                   torch.cuda.current_stream())
    assert ring.host_dev_ptr is not None, "the pinned ring is not mapped for the device"
    for i, o in enumerate(outs):
        assert torch.equal(o, refs[i % 3]), f"call {i} differs"


def test_group_tables_on_two_streams():
    """Each stream stages its calls' group tables in its own pinned ring.
    Decode calls alternating between two side streams (no sync between
    them, 600 calls of 129 table words each, so both rings wrap) match the
    device-id results bit for bit."""
    from nf4_grouped import gemm_4bit_grouped
    W, S = _stack("nf4", 32, 256, 512, seed=95)
    g = torch.Generator().manual_seed(96)
    sizes = torch.randint(1, 4, (64,), generator=g).tolist()
    ids = [torch.randint(0, 32, (64,), generator=g).tolist() for _ in range(2)]
    a = rand_acts(sum(sizes), 512, seed=97)
    refs = [gemm_4bit_grouped(a, W, S, sizes, torch.tensor(i, dtype=torch.int32, device="cuda"))
            for i in ids]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s_ in streams:
        s_.wait_stream(torch.cuda.current_stream())
    outs = [[], []]
    for i in range(1200):
        j = i % 2
        with torch.cuda.stream(streams[j]):
            outs[j].append(gemm_4bit_grouped(a, W, S, sizes, ids[j]))
    torch.cuda.synchronize()
    for j in range(2):
        for i, o in enumerate(outs[j]):
            assert torch.equal(o, refs[j]), (j, i)


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_op_captures_after_one_eager_call(fmt):
    """An eager call (tables through the staging rings) followed by a graph
    capture of the same op (tables through the capture-safe pinned arena,
    which the eager call must have created): the capture succeeds and its
    replays give the eager bits, for the decode and the tiled paths."""
    import nf4_grouped
    op = _ops()[fmt]
    W, S = _stack(fmt, 8, 256, 512, seed=95)
    # as in a fresh process: no arena yet (earlier tests' arenas are set
    # aside, not freed, and restored afterwards)
    saved = dict(nf4_grouped._ARENAS)
    nf4_grouped._ARENAS.clear()
    graphs = []
    try:
        for sizes, ids in (([2, 1, 3], [1, 5, 7]), ([40, 300, 7], [2, 4, 6])):
            a = rand_acts(sum(sizes), 512, seed=96)
            eager = op(a, W, S, sizes, ids)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = op(a, W, S, sizes, ids)
            graphs.append(graph)
            for _ in range(3):
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, eager)
    finally:
        torch.cuda.synchronize()
        fresh = dict(nf4_grouped._ARENAS)
        del graphs
        nf4_grouped._ARENAS.clear()
        nf4_grouped._ARENAS.update(saved)
        del fresh
