"""Pin the CPU oracle (oracle/) before trusting it as the GPU checker.

What pins what (reference files cited inline):
  * codebooks   -- the reference's literal values; transformers' FP4_VALUES.
  * decode      -- closed-form nibble order over all 256 bytes; MXFP4 byte
                   0x21 known answer; transformers' own MXFP4 dequant; e8m0
                   0x00 / 0xFF edges.
  * locked tree -- C oracle == numpy spec == the reference's compiled CPU
                   kernels (oracle/_ref) == the golden vectors those kernels
                   wrote (tests/golden), bit for bit; thread count invariance;
                   an independent fp64 check (catches a shared misreading).
  * packers     -- argmin / first-index-on-ties by brute force; round trip.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import native, spec

GOLDEN = Path(__file__).resolve().parent / "golden"

E, N, K = 4, 24, 128
SIZES = [1, 2, 1]
EIDS = [2, 0, 3]

# the reference's literal codebooks, kernel/nf4_grouped.py:53-70 and
# kernel/mxfp4_pack_ref.py:21-22
NF4_REF = [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
           -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
           0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
           0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
           0.7229568362236023, 1.0]
FP4_REF = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
           -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def nanfix(x):
    return np.nan_to_num(np.asarray(x), nan=1e30, posinf=2e30, neginf=-2e30)


def nf4_stack(seed, rows, k=K):
    g = np.random.default_rng(seed)
    packed = g.integers(0, 256, size=(E, N, k // 2), dtype=np.uint8)
    absmax = g.random(size=(E, N, k // 64), dtype=np.float32) + 0.5
    a = g.standard_normal((rows, k), dtype=np.float32)
    return a, packed, absmax


def mx_stack(seed, rows, weird=False, k=K):
    g = np.random.default_rng(seed)
    packed = g.integers(0, 256, size=(E, N, k // 2), dtype=np.uint8)
    scales = g.integers(100, 140, size=(E, N, k // 32), dtype=np.uint8)
    if weird:
        scales[0, 0, 0] = 0xFF
        scales[0, 0, 1] = 0
        scales[1, 3, scales.shape[2] - 1] = 0xFF
    a = g.standard_normal((rows, k), dtype=np.float32)
    return a, packed, scales


# ---------------------------------------------------------------- codebooks --

def test_codebooks_match_the_reference_literals_everywhere():
    import mxfp4_grouped
    import mxfp4_pack_ref
    import nf4_grouped
    nf4_c, fp4_c = native.oracle_luts()
    want_nf4 = np.asarray(NF4_REF, dtype=np.float32)
    want_fp4 = np.asarray(FP4_REF, dtype=np.float32)
    for got in (nf4_c, spec.NF4_LUT32, np.asarray(nf4_grouped.NF4_LUT, np.float32)):
        assert np.array_equal(got.view(np.uint32), want_nf4.view(np.uint32))
    for got in (fp4_c, spec.FP4_LUT32, np.asarray(mxfp4_grouped.FP4_VALUES, np.float32),
                np.asarray(mxfp4_pack_ref.FP4_VALUES, np.float32)):
        assert np.array_equal(got.view(np.uint32), want_fp4.view(np.uint32))  # -0.0 too
    assert nf4_grouped.BLOCKSIZE == spec.BLOCKSIZE == 64
    assert mxfp4_grouped.MX_BLOCK == spec.MX_BLOCK == 32 and mxfp4_grouped.E8M0_BIAS == 127
    assert spec.NF4_LUT32[7] == 0.0 and np.all(np.diff(spec.NF4_LUT32) > 0)


def test_fp4_codebook_matches_transformers():
    M = pytest.importorskip("transformers.integrations.mxfp4")
    assert list(M.FP4_VALUES) == FP4_REF


# ------------------------------------------------------------------- decode --

def test_nibble_order_closed_form_over_all_bytes():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256)
    nf = spec.codes_nf4(b)[0]
    mx = spec.codes_mxfp4(b)[0]
    for v in range(256):
        assert (nf[2 * v], nf[2 * v + 1]) == (v >> 4, v & 15)     # NF4: 2j = HIGH
        assert (mx[2 * v], mx[2 * v + 1]) == (v & 15, v >> 4)     # MXFP4: 2j = LOW


def test_mxfp4_byte_0x21_known_answer():
    # reference kernel/test_mxfp4_oracle.py:51-71: low nibble 1 -> 0.5, high 2 -> 1.0
    blocks = np.zeros((1, 16), dtype=np.uint8)
    blocks[0, 0] = 0x21
    w = spec.dequant_mxfp4(blocks, np.full((1, 1), 127, np.uint8))
    assert (w[0, 0], w[0, 1]) == (0.5, 1.0) and not np.any(w[0, 2:])


def test_e8m0_edges():
    blocks = np.full((1, 16), 0x21, dtype=np.uint8)
    w0 = spec.dequant_mxfp4(blocks, np.zeros((1, 1), np.uint8))
    assert w0[0, 0] == np.float32(2.0 ** -128) and w0[0, 1] == np.float32(2.0 ** -127)
    blocks[0, 1] = 0x00
    with np.errstate(over="ignore"):
        wf = spec.dequant_mxfp4(blocks, np.full((1, 1), 255, np.uint8))
    # 0.5 * 2^128 = 2^127 is finite, 1.0 * 2^128 overflows; ldexp keeps 0 at 0
    assert wf[0, 0] == np.float32(2.0 ** 127) and np.isinf(wf[0, 1])
    assert wf[0, 2] == 0.0 and wf[0, 3] == 0.0


def test_nf4_decode_is_one_rounding_of_lut_times_absmax():
    g = np.random.default_rng(3)
    packed = g.integers(0, 256, size=(5, 96), dtype=np.uint8)
    absmax = (g.random(size=(5, 3)) * 10).astype(np.float32)
    w = spec.dequant_nf4(packed, absmax)
    for r in range(5):
        for k in range(192):
            byte = packed[r, k // 2]
            c = byte >> 4 if k % 2 == 0 else byte & 15
            assert w[r, k] == np.float32(NF4_REF[c]) * absmax[r, k // 64]


@pytest.mark.parametrize("seed", [0, 1, 7])
def test_mxfp4_decode_matches_transformers(seed):
    torch = pytest.importorskip("torch")
    M = pytest.importorskip("transformers.integrations.mxfp4")
    fn = getattr(M, "_convert_moe_packed_tensors", None)
    if fn is None:
        pytest.skip("transformers lacks _convert_moe_packed_tensors")
    g = np.random.default_rng(seed)
    blocks = g.integers(0, 256, size=(3, 4, 16), dtype=np.uint8)
    scales = g.integers(115, 140, size=(3, 4), dtype=np.uint8)
    ref = fn(torch.from_numpy(blocks).unsqueeze(0), torch.from_numpy(scales).unsqueeze(0),
             dtype=torch.float32, rows_per_chunk=1 << 30)
    ref = ref.transpose(1, 2).reshape(3, 4 * 32).numpy()
    ours = spec.dequant_mxfp4(blocks.reshape(3, 64), scales)
    assert np.array_equal(ours, ref)


def test_package_reference_decoders_match_the_spec():
    torch = pytest.importorskip("torch")
    from mxfp4_pack_ref import dequant_mxfp4
    from nf4_grouped import dequant_ref
    g = np.random.default_rng(11)
    packed = g.integers(0, 256, size=(7, 64), dtype=np.uint8)
    absmax = (g.random(size=(7, 2)) + 0.1).astype(np.float32)
    got = dequant_ref(torch.from_numpy(packed), torch.from_numpy(absmax), 7, 128).numpy()
    assert np.array_equal(got, spec.dequant_nf4(packed, absmax))
    scales = g.integers(90, 160, size=(7, 4), dtype=np.uint8)
    got = dequant_mxfp4(torch.from_numpy(packed.reshape(7, 4, 16)), torch.from_numpy(scales)).numpy()
    assert np.array_equal(got, spec.dequant_mxfp4(packed, scales))


# -------------------------------------------------------------- locked tree --

def test_c_oracle_equals_numpy_spec_nf4():
    a, p, s = nf4_stack(0, sum(SIZES))
    assert np.array_equal(native.gemv_grouped(a, p, s, SIZES, EIDS, fmt="nf4"),
                          spec.ref_gemv_grouped(a, p, s, SIZES, EIDS, fmt="nf4"))


@pytest.mark.parametrize("weird", [False, True])
def test_c_oracle_equals_numpy_spec_mxfp4(weird):
    a, p, s = mx_stack(1, sum(SIZES), weird)
    with np.errstate(over="ignore"):
        want = spec.ref_gemv_grouped(a, p, s, SIZES, EIDS, fmt="mxfp4")
    assert np.array_equal(nanfix(native.gemv_grouped(a, p, s, SIZES, EIDS, fmt="mxfp4")), nanfix(want))


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
@pytest.mark.parametrize("sizes", [[9], [16], [8, 17, 1], [33, 2], [3, 0, 5]])
def test_large_and_empty_groups_equal_the_spec(fmt, sizes):
    eids = [i % E for i in range(len(sizes))]
    a, p, s = (nf4_stack(0, sum(sizes)) if fmt == "nf4" else mx_stack(1, sum(sizes)))
    assert np.array_equal(native.gemv_grouped(a, p, s, sizes, eids, fmt=fmt),
                          spec.ref_gemv_grouped(a, p, s, sizes, eids, fmt=fmt))


@pytest.mark.parametrize("k", [64, 128, 192, 320])
@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_c_oracle_equals_spec(fmt, k):
    _, p, s = nf4_stack(17, 1, k=k) if fmt == "nf4" else mx_stack(17, 1, weird=True, k=k)
    g = np.random.default_rng(k).standard_normal((sum(SIZES), N), dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        want = spec.ordered_dgrad_ref(g, p, s, SIZES, EIDS, fmt=fmt)
    got = native.dgrad_grouped(g, p, s, SIZES, EIDS, fmt=fmt)
    assert np.array_equal(nanfix(got), nanfix(want))


def test_thread_count_does_not_change_bits():
    a, p, s = nf4_stack(7, 40)
    sizes, eids = [13, 20, 7], [1, 3, 0]
    one = native.gemv_grouped(a, p, s, sizes, eids, fmt="nf4", threads=1)
    four = native.gemv_grouped(a, p, s, sizes, eids, fmt="nf4", threads=4)
    assert np.array_equal(one, four)
    g = np.random.default_rng(8).standard_normal((40, N), dtype=np.float32)
    assert np.array_equal(native.dgrad_grouped(g, p, s, sizes, eids, fmt="nf4", threads=1),
                          native.dgrad_grouped(g, p, s, sizes, eids, fmt="nf4", threads=3))


def _golden_cases():
    return sorted(GOLDEN.glob("*.npz"))


@pytest.mark.parametrize("path", _golden_cases(), ids=lambda p: p.stem)
def test_c_oracle_reproduces_the_reference_golden_vectors(path):
    """Vectors written by the reference's compiled CPU kernels."""
    z = np.load(path)                       # allow_pickle stays False
    op = str(z["op"])
    if op == "route":
        k, mode, norm = int(z["k"]), int(z["mode"]), int(z["norm"])
        idx, wts = native.route_topk(z["logits"], k, mode, norm)
        assert np.array_equal(idx, z["idx"]) and np.array_equal(wts, z["wts"])
        return
    fmt = str(z["fmt"])
    sizes, eids = z["sizes"].tolist(), z["eids"].tolist()
    if op == "ffn":
        args = (z["x"], z["gu_packed"], z["gu_absmax"], z["dn_packed"], z["dn_absmax"],
                sizes, eids)
        assert np.array_equal(native.ffn_grouped(*args), z["out"])
        assert np.array_equal(spec.ref_ffn_grouped(*args), z["out"])
        return
    fn = native.gemv_grouped if op == "gemv" else native.dgrad_grouped
    got = fn(z["x"], z["packed"], z["scales"], sizes, eids, fmt=fmt)
    assert np.array_equal(nanfix(got), nanfix(z["out"]))


def test_golden_set_is_complete():
    names = {p.stem for p in _golden_cases()}
    assert {"gemv_nf4_fixture", "gemv_mxfp4_weird_scales", "dgrad_nf4_fixture",
            "dgrad_mxfp4_weird_scales", "gemv_nf4_config1_slice", "ffn_nf4_groups_1_9_3",
            "ffn_nf4_single_rows", "ffn_nf4_groups_8_8", "ffn_nf4_silu_clamps",
            "route_tie_mode0", "route_tie_mode0_norm", "route_tie_mode1",
            "route_qwen3_top8_norm", "route_gptoss_top4"} <= names


needs_ref = pytest.mark.skipif(native.ref_lib() is None, reason="oracle/_ref not built here")


@needs_ref
@pytest.mark.parametrize("seed", [0, 5, 9])
@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_c_oracle_equals_the_compiled_reference_live(fmt, seed):
    rng = np.random.default_rng(seed)
    sizes = [int(x) for x in rng.integers(1, 12, size=5)]
    eids = [int(x) for x in rng.integers(0, E, size=5)]
    a, p, s = nf4_stack(seed, sum(sizes), k=256) if fmt == "nf4" else mx_stack(seed, sum(sizes), True, k=256)
    got = native.gemv_grouped(a, p, s, sizes, eids, fmt=fmt)
    ref = native.ref_gemv_grouped(a, p, s, sizes, eids, fmt=fmt)
    assert np.array_equal(nanfix(got), nanfix(ref))
    g = rng.standard_normal((sum(sizes), N), dtype=np.float32)
    assert np.array_equal(nanfix(native.dgrad_grouped(g, p, s, sizes, eids, fmt=fmt)),
                          nanfix(native.ref_dgrad_grouped(g, p, s, sizes, eids, fmt=fmt)))


# ---------------------------------------------- independent fp64 agreement --

@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_forward_agrees_with_fp64(fmt):
    a, p, s = nf4_stack(3, 20, k=512) if fmt == "nf4" else mx_stack(3, 20, k=512)
    sizes, eids = [6, 9, 5], [0, 2, 3]
    got = native.gemv_grouped(a, p, s, sizes, eids, fmt=fmt)
    want = spec.fp64_forward(a, p, s, sizes, eids, fmt=fmt)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5 * np.abs(want).max())


@pytest.mark.parametrize("fmt", ["nf4", "mxfp4"])
def test_dgrad_is_the_forward_transpose(fmt):
    """<dX, x> == <dY, W x> per group in fp64: a transposed or mis-indexed
    dgrad fails this, whatever the summation order."""
    _, p, s = nf4_stack(11, 1, k=256) if fmt == "nf4" else mx_stack(11, 1, k=256)
    sizes, eids = [4, 7], [1, 3]
    rng = np.random.default_rng(12)
    dy = rng.standard_normal((11, N), dtype=np.float32)
    x = rng.standard_normal((11, 256), dtype=np.float32)
    dx = native.dgrad_grouped(dy, p, s, sizes, eids, fmt=fmt).astype(np.float64)
    wx = spec.fp64_forward(x, p, s, sizes, eids, fmt=fmt)
    lhs = np.sum(dx * x.astype(np.float64))
    rhs = np.sum(dy.astype(np.float64) * wx)
    assert abs(lhs - rhs) <= 1e-4 * (abs(rhs) + 1)


def test_one_hot_rows_reduce_to_the_decode():
    """A one-hot activation turns the locked tree into a single product: the
    output is the decoded weight exactly."""
    _, p, s = nf4_stack(21, 1, k=256)
    a = np.zeros((3, 256), dtype=np.float32)
    cols = [0, 131, 255]
    for r, c in enumerate(cols):
        a[r, c] = 1.0
    out = native.gemv_grouped(a, p, s, [3], [2], fmt="nf4")
    w = spec.dequant_nf4(p[2], s[2])
    for r, c in enumerate(cols):
        assert np.array_equal(out[r], w[:, c])


# ------------------------------------------------------------------ packers --

def test_nf4_packer_is_nearest_code_first_index_on_ties():
    torch = pytest.importorskip("torch")
    from nf4_pack_ref import quantize_pack_nf4
    g = torch.Generator().manual_seed(0)
    w = torch.randn(6, 128, generator=g)
    w[0, 5] = 0.0                 # exact code 7
    w[1, :64] = 0.0               # all-zero block -> absmax clamp
    packed, absmax = quantize_pack_nf4(w)
    assert absmax[1, 0].item() == pytest.approx(1e-12)
    lut = np.asarray(NF4_REF, np.float32)
    codes = spec.codes_nf4(packed.numpy())
    am = absmax.numpy()
    for r in range(6):
        for k in range(128):
            x = np.float32(w[r, k].item()) / am[r, k // 64]
            d = np.abs(np.float32(x) - lut)
            assert codes[r, k] == int(np.argmin(d))     # numpy argmin: first index on ties
    assert codes[0, 5] == 7


def test_packers_round_trip():
    torch = pytest.importorskip("torch")
    from mxfp4_pack_ref import dequant_mxfp4, quantize_pack_mxfp4
    from nf4_grouped import dequant_ref
    from nf4_pack_ref import quantize_pack_nf4
    g = torch.Generator().manual_seed(1)
    w = torch.randn(64, 256, generator=g)
    p, a = quantize_pack_nf4(w)
    rel = ((dequant_ref(p, a, 64, 256) - w).norm() / w.norm()).item()
    assert 0.05 < rel < 0.12          # reference README: ~0.09
    b, s = quantize_pack_mxfp4(w)
    rel = ((dequant_mxfp4(b, s) - w).norm() / w.norm()).item()
    assert 0.05 < rel < 0.16          # reference README: ~0.12
    assert (s.int() - 127).abs().max().item() <= 127


# ------------------------------------------------------- fused FFN (silu) --

def test_silu_locked_tracks_true_silu_and_its_tails():
    """The locked sequence is silu: within 2e-6 relative of float64
    x / (1 + exp(-x)) on the clamped domain (the reference's own diagnostic
    bound, kernel/test_cpu_grouped.py:406-424), exactly x above 87 and exactly
    0 below -87."""
    x = np.linspace(-87.0, 87.0, 20011, dtype=np.float32)
    got = spec.silu_locked(x)
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-6)) < 2e-6
    big = np.asarray([87.5, 88.0, 500.0, 1e30, np.inf], dtype=np.float32)
    assert np.array_equal(spec.silu_locked(big), big)
    assert np.array_equal(spec.silu_locked(-big), np.zeros_like(big))
    assert spec.silu_locked(np.float32(0.0)) == 0.0


def test_silu_c_oracle_equals_the_numpy_spec_bitwise():
    rng = np.random.default_rng(3)
    x = np.concatenate([np.linspace(-100, 100, 100001, dtype=np.float32),
                        rng.standard_normal(50000).astype(np.float32) * 30,
                        np.asarray([-87, 87, -86.99999, 86.99999, 1e-30, -1e-30], np.float32)])
    assert np.array_equal(native.silu_locked(x), spec.silu_locked(x))


def test_ffn_oracle_is_the_composition_of_its_parts():
    """gemv -> silu_locked(gate) * up -> gemv, each part the oracle's own."""
    a, gu_p, gu_a, dn_p, dn_a, sizes, eids = _ffn_case(31, (4, 7))
    gu = native.gemv_grouped(a, gu_p, gu_a, sizes, eids, fmt="nf4")
    h = spec.silu_locked(gu[:, :64]) * gu[:, 64:]
    dn = native.gemv_grouped(h, dn_p, dn_a, sizes, eids, fmt="nf4")
    assert np.array_equal(native.ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, eids), dn)


def test_ffn_oracle_agrees_with_fp64():
    a, gu_p, gu_a, dn_p, dn_a, sizes, eids = _ffn_case(32, (3, 6, 2))
    got = native.ffn_grouped(a, gu_p, gu_a, dn_p, dn_a, sizes, eids)
    want = spec.fp64_ffn(a, gu_p, gu_a, dn_p, dn_a, sizes, eids)
    assert spec.rel_fro(got, want) < 1e-5


def test_ffn_oracle_rejects_bad_shapes():
    a, gu_p, gu_a, dn_p, dn_a, sizes, eids = _ffn_case(33, (2,))
    with pytest.raises(ValueError):          # odd gu width
        native.ffn_grouped(a, gu_p[:, :-1], gu_a[:, :-1], dn_p, dn_a, sizes, eids)
    with pytest.raises(ValueError):          # H % 64 != 0
        native.ffn_grouped(a, gu_p[:, :96], gu_a[:, :96], dn_p[:, :, :24], dn_a, sizes, eids)


def _ffn_case(seed, sizes, scale=1.0):
    g = np.random.default_rng(seed)
    gu_p = g.integers(0, 256, size=(E, 128, 64), dtype=np.uint8)
    gu_a = (g.random(size=(E, 128, 2), dtype=np.float32) + 0.5) * np.float32(scale)
    dn_p = g.integers(0, 256, size=(E, 24, 32), dtype=np.uint8)
    dn_a = g.random(size=(E, 24, 1), dtype=np.float32) + 0.5
    a = g.standard_normal((sum(sizes), 128), dtype=np.float32)
    return a, gu_p, gu_a, dn_p, dn_a, list(sizes), [int(x) for x in g.permutation(E)[:len(sizes)]]


@needs_ref
@pytest.mark.parametrize("sizes,scale", [((1, 9, 3), 1.0), ((1, 1, 1, 1), 1.0),
                                         ((8, 8), 1.0), ((2, 5), 40.0), ((12, 3, 1), 7.0)])
def test_ffn_oracle_equals_the_compiled_reference_live(sizes, scale):
    args = _ffn_case(40 + len(sizes), sizes, scale)
    assert np.array_equal(native.ffn_grouped(*args), native.ref_ffn_grouped(*args))


# ---------------------------------------------------------------- routing --

@pytest.mark.parametrize("t,e,k", [(3, 64, 8), (40, 128, 8), (25, 32, 4), (5, 300, 64)])
def test_route_selection_is_the_stable_descending_sort(t, e, k):
    rng = np.random.default_rng(t + e)
    lg = rng.standard_normal((t, e)).astype(np.float32)
    lg[0, 2] = lg[0, 7] = lg[0, 1]                       # ties
    lg[1, :] = 0.5                                       # all equal
    for mode, norm in ((0, 0), (0, 1), (1, 0)):
        idx, wts = native.route_topk(lg, k, mode, norm)
        assert np.array_equal(idx, np.argsort(-lg, axis=-1, kind="stable")[:, :k])


def test_route_weights_follow_the_softmax_closed_forms():
    rng = np.random.default_rng(9)
    lg = (rng.standard_normal((30, 128)) * 3).astype(np.float32)
    k = 8
    order = np.argsort(-lg, axis=-1, kind="stable")[:, :k]
    top = np.take_along_axis(lg, order, -1).astype(np.float64)
    full = np.exp(lg - lg.max(-1, keepdims=True))
    full = full / full.sum(-1, keepdims=True)
    sel = np.take_along_axis(full, order, -1)
    want = {(0, 0): sel, (0, 1): sel / sel.sum(-1, keepdims=True),
            (1, 0): np.exp(top - top[:, :1]) / np.exp(top - top[:, :1]).sum(-1, keepdims=True)}
    for (mode, norm), w in want.items():
        _idx, wts = native.route_topk(lg, k, mode, norm)
        got = (wts.astype(np.uint32) << 16).view(np.float32)
        np.testing.assert_allclose(got, w, rtol=8e-3, atol=1e-6)


@needs_ref
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_route_topk_equals_the_compiled_reference_live(seed):
    rng = np.random.default_rng(seed)
    lg = (rng.standard_normal((33, 128)) * (1 + seed)).astype(np.float32)
    lg[3, 10] = lg[3, 20] = lg[3, 30]
    for k, mode, norm in ((8, 0, 1), (8, 0, 0), (4, 1, 0), (64, 0, 1)):
        a = native.route_topk(lg, k, mode, norm)
        b = native.ref_route_topk(lg, k, mode, norm)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_route_groups_is_the_stable_sort_by_expert():
    rng = np.random.default_rng(4)
    for T, k, E in ((1, 8, 128), (16, 8, 128), (300, 4, 32), (7, 2, 3)):
        ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
        eids, row_off, order, pos = native.route_groups(ids, E)
        flat = ids.reshape(-1)
        want_order = np.argsort(flat, kind="stable")
        assert np.array_equal(order, want_order)
        assert np.array_equal(pos[order], np.arange(flat.size))
        counts = np.bincount(flat, minlength=E)
        assert np.array_equal(eids, np.nonzero(counts)[0])
        assert np.array_equal(np.diff(row_off), counts[counts > 0])
        assert row_off[0] == 0 and row_off[-1] == flat.size
    with pytest.raises(ValueError):
        native.route_groups(np.array([[0, 5]]), 4)
