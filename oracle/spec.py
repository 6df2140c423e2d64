"""numpy executable spec of the reference's locked CPU summation order.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates reference kernel/cpu_grouped.py:53-144 (``ordered_dot``,
``dequant_row_nf4``, ``dequant_row_mxfp4``, ``ref_gemv_grouped``,
``ordered_dgrad_ref``) with the same arithmetic, vectorised across output
elements -- numpy float32 elementwise ops are single IEEE roundings, so
vectorising across independent outputs cannot change a bit, only the per-
element operation order matters and that is kept.
"""
from __future__ import annotations

import numpy as np

BLOCKSIZE = 64   # NF4 absmax block (reference kernel/nf4_grouped.py:71)
MX_BLOCK = 32    # MXFP4 e8m0 block (reference kernel/mxfp4_pack_ref.py:23)

# reference kernel/nf4_grouped.py:53-70
NF4_LUT32 = np.asarray([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
    0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0,
], dtype=np.float32)

# reference kernel/mxfp4_pack_ref.py:21-22
FP4_LUT32 = np.asarray([
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
], dtype=np.float32)


def codes_nf4(packed: np.ndarray) -> np.ndarray:
    """[..., K/2] u8 -> [..., K] codes; element 2j = HIGH nibble
    (reference kernel/nf4_grouped.py:918-920)."""
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed >> 4
    out[..., 1::2] = packed & 0x0F
    return out


def codes_mxfp4(packed: np.ndarray) -> np.ndarray:
    """[..., K/2] u8 -> [..., K] codes; element 2j = LOW nibble
    (reference kernel/mxfp4_pack_ref.py:25-29)."""
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 0x0F
    out[..., 1::2] = packed >> 4
    return out


def dequant_nf4(packed: np.ndarray, absmax: np.ndarray) -> np.ndarray:
    """w = LUT[code] * absmax[k // 64] in fp32, one rounding
    (reference kernel/cpu_grouped.py:75-84)."""
    codes = codes_nf4(packed)
    scale = np.repeat(absmax.astype(np.float32), BLOCKSIZE, axis=-1)
    return (NF4_LUT32[codes] * scale).astype(np.float32)


def e8m0_scale32(scales: np.ndarray) -> np.ndarray:
    """2^(e-127) as float32 for e in 0..254; e = 255 maps to +inf here and is
    handled with ldexp semantics by ``dequant_mxfp4``."""
    return np.ldexp(np.float32(1.0), scales.astype(np.int32) - 127).astype(np.float32)


def dequant_mxfp4(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """w = ldexp(FP4[code], e - 127) in fp32 (reference kernel/cpu_grouped.py:
    87-96; ldexp keeps zero at zero for e = 255)."""
    codes = codes_mxfp4(packed)
    exp = np.repeat(scales.astype(np.int32) - 127, MX_BLOCK, axis=-1)
    return np.ldexp(FP4_LUT32[codes], exp).astype(np.float32)


def dequant(fmt: str, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    return dequant_nf4(packed, scales) if fmt == "nf4" else dequant_mxfp4(packed, scales)


def ordered_dot_rows(a32: np.ndarray, w32: np.ndarray) -> np.ndarray:
    """The locked tree for every (row, column) pair at once.

    a32 [R, K], w32 [C, K] -> [R, C]. Per output element: 16-lane groups in
    ascending order, lane group g into accumulator g % 4, separate multiply
    and add, combine (acc0 + acc1) + (acc2 + acc3), then a sequential sum of
    the 16 lanes (reference kernel/cpu_grouped.py:53-72)."""
    assert a32.dtype == np.float32 and w32.dtype == np.float32
    R, K = a32.shape
    C = w32.shape[0]
    assert K % 16 == 0
    acc = np.zeros((4, R, C, 16), dtype=np.float32)
    a3 = a32.reshape(R, K // 16, 16)
    w3 = w32.reshape(C, K // 16, 16)
    with np.errstate(invalid="ignore", over="ignore"):
        for g in range(K // 16):
            prod = w3[None, :, g, :] * a3[:, None, g, :]       # [R, C, 16]
            acc[g % 4] = acc[g % 4] + prod
        comb = (acc[0] + acc[1]) + (acc[2] + acc[3])           # [R, C, 16]
        s = np.zeros((R, C), dtype=np.float32)
        for i in range(16):
            s = s + comb[:, :, i]
    return s


def ref_gemv_grouped(a32, packed, scales, sizes, expert_ids, *, fmt):
    """Full forward spec: bit-identical to the reference's native CPU kernel
    (reference kernel/cpu_grouped.py:99-116). fp32 [R, N]."""
    assert fmt in ("nf4", "mxfp4")
    n = packed.shape[1]
    out = np.empty((a32.shape[0], n), dtype=np.float32)
    r = 0
    for g, e in enumerate(expert_ids):
        m = int(sizes[g])
        if m:
            w = dequant(fmt, packed[e], scales[e])
            out[r:r + m] = ordered_dot_rows(a32[r:r + m], w)
        r += m
    return out


def ordered_dgrad_ref(g32, packed, scales, sizes, expert_ids, *, fmt):
    """dgrad spec: gi[t, k] = fold over n ascending of (w[n, k] * g[t, n]),
    separate multiply and add (reference kernel/cpu_grouped.py:119-144)."""
    assert fmt in ("nf4", "mxfp4")
    n_cols = packed.shape[1]
    k = packed.shape[2] * 2
    out = np.zeros((g32.shape[0], k), dtype=np.float32)
    r = 0
    with np.errstate(invalid="ignore", over="ignore"):
        for gi, e in enumerate(expert_ids):
            m = int(sizes[gi])
            if m:
                w = dequant(fmt, packed[e], scales[e])          # [N, K]
                blk = out[r:r + m]
                for n in range(n_cols):
                    blk[:] = blk + w[n][None, :] * g32[r:r + m, n][:, None]
            r += m
    return out


# Horner coefficients of the locked silu, highest degree first, and the
# clamp (reference kernel/cpu_grouped.py:147-179, gnf4_native/cpu_kernels.c:789-795).
SILU_HORNER = (1.535336188319500e-4, 1.339887440266574e-3, 9.618437357674640e-3,
               5.550332471162809e-2, 2.402264791363012e-1, 6.931472028550421e-1, 1.0)
SILU_CLAMP = 87.0


def silu_locked(x):
    """The fused FFN's fp32 silu as its fixed op sequence, vectorised: every
    step below is one IEEE fp32 operation per element, in the reference's
    order (clamp, t = x * -log2(e), n = floor(t + 0.5), f = t - n, Horner with
    separate multiply and add, e = p * 2^n, 1 / (1 + e), x * that), with the
    exact tails x (x > 87) and 0 (x < -87)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        xc = np.clip(x, np.float32(-SILU_CLAMP), np.float32(SILU_CLAMP))
        t = xc * np.float32(-1.442695040888963e0)
        n = np.floor(t + np.float32(0.5))
        f = t - n
        p = np.full_like(f, np.float32(SILU_HORNER[0]))
        for c in SILU_HORNER[1:]:
            p = p * f + np.float32(c)
        two_n = ((n.astype(np.int32) + 127).astype(np.uint32) << 23).view(np.float32)
        e = p * two_n
        r = x * (np.float32(1.0) / (np.float32(1.0) + e))
    r = np.where(x > np.float32(SILU_CLAMP), x, r)
    return np.where(x < np.float32(-SILU_CLAMP), np.float32(0.0), r).astype(np.float32)


def ref_ffn_grouped(a32, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes, expert_ids):
    """Fused NF4 FFN spec: forward spec -> silu_locked(gate) * up -> forward
    spec, gate = the first H outputs, up = the last H (reference
    kernel/cpu_grouped.py:182-194)."""
    gu = ref_gemv_grouped(a32, gu_packed, gu_absmax, sizes, expert_ids, fmt="nf4")
    h_dim = gu.shape[1] // 2
    h = silu_locked(gu[:, :h_dim]) * gu[:, h_dim:]
    return ref_gemv_grouped(h, dn_packed, dn_absmax, sizes, expert_ids, fmt="nf4")


def fp64_ffn(a, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes, expert_ids):
    """The FFN in float64 with the exact silu x / (1 + exp(-x))."""
    gu = fp64_forward(a, gu_packed, gu_absmax, sizes, expert_ids, fmt="nf4")
    h_dim = gu.shape[1] // 2
    gate = gu[:, :h_dim]
    with np.errstate(over="ignore"):
        h = gate / (1.0 + np.exp(-gate)) * gu[:, h_dim:]
    return fp64_forward(h, dn_packed, dn_absmax, sizes, expert_ids, fmt="nf4")


def fp64_forward(a, packed, scales, sizes, expert_ids, *, fmt):
    """out = a @ dequant(W[e]).T per group in float64 (the tolerance
    contract's reference, reference docs/TOLERANCE_CONTRACT.md)."""
    a = np.asarray(a, dtype=np.float64)
    n = packed.shape[1]
    out = np.zeros((a.shape[0], n), dtype=np.float64)
    r = 0
    for g, e in enumerate(expert_ids):
        m = int(sizes[g])
        if m:
            w = dequant(fmt, packed[e], scales[e]).astype(np.float64)
            out[r:r + m] = a[r:r + m] @ w.T
        r += m
    return out


def fp64_dgrad(g, packed, scales, sizes, expert_ids, *, fmt):
    """gi = g @ dequant(W[e]) per group in float64."""
    g = np.asarray(g, dtype=np.float64)
    k = packed.shape[2] * 2
    out = np.zeros((g.shape[0], k), dtype=np.float64)
    r = 0
    for gi, e in enumerate(expert_ids):
        m = int(sizes[gi])
        if m:
            w = dequant(fmt, packed[e], scales[e]).astype(np.float64)
            out[r:r + m] = g[r:r + m] @ w
        r += m
    return out


def rel_fro(x, ref) -> float:
    """||x - ref||_F / ||ref||_F in float64."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(x - ref) / max(den, 1e-300))
