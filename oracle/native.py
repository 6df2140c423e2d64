"""ctypes bindings to the C oracle and to the compiled reference.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``liboracle.so``      -- ``gnf4_oracle.c`` in this directory (built by
  ``make -C oracle``); restates the reference's locked tree.
* ``_ref/libgnf4_ref_v{3,4}.so`` -- the reference's gnf4_native/cpu_kernels.c
  compiled from its own source by ``oracle/Makefile``; used as an independent
  check of the restatement and as the timed CPU baseline. The v4 build needs
  AVX-512; the loader picks the highest level the running CPU supports.

The reference entry points keep its ABI (reference gnf4_native/build.py:103-147):
``gnf4_gemv_{nf4,mxfp4}_grouped`` and ``gnf4_dgrad_{nf4,mxfp4}_grouped`` take
(a, B, scales, eids i64[G], sizes i32[G], G, N i64, K i64, out, threads) and
reject G > 512 or a size < 1.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
FMT = {"nf4": 0, "mxfp4": 1}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _cpu_has_avx512() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl", "avx512cd"))


_lib = None
_ref = None
_ref_path = None


def oracle_lib():
    """The C oracle; raises with a build hint if it was not built."""
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        lib = ctypes.CDLL(str(path))
        for name in ("gnf4o_gemv_grouped", "gnf4o_dgrad_grouped"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.c_int, _P, _P, _P, _P, _P, ctypes.c_int,
                           _I64, _I64, _I64, _P, ctypes.c_int]
        lib.gnf4o_silu_locked.restype = None
        lib.gnf4o_silu_locked.argtypes = [_P, _P, _I64]
        lib.gnf4o_ffn_grouped.restype = ctypes.c_int
        lib.gnf4o_ffn_grouped.argtypes = [_P, _P, _P, _P, _P, _P, _P, ctypes.c_int,
                                          _I64, _I64, _I64, _I64, _P, ctypes.c_int]
        lib.gnf4o_route_topk.restype = ctypes.c_int
        lib.gnf4o_route_topk.argtypes = [_P, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int,
                                         _P, _P]
        lib.gnf4o_route_groups.restype = ctypes.c_int
        lib.gnf4o_route_groups.argtypes = [_P, _I64, _I64, _P, _P, _P, _P]
        lib.gnf4o_nf4_lut.restype = ctypes.POINTER(ctypes.c_float)
        lib.gnf4o_fp4_lut.restype = ctypes.POINTER(ctypes.c_float)
        _lib = lib
    return _lib


def ref_lib():
    """The compiled reference (or None when it was not built here)."""
    global _ref, _ref_path
    if _ref is None:
        cands = []
        if _cpu_has_avx512():
            cands.append(HERE / "_ref" / "libgnf4_ref_v4.so")
        cands.append(HERE / "_ref" / "libgnf4_ref_v3.so")
        for path in cands:
            if path.exists():
                lib = ctypes.CDLL(str(path))
                for name in ("gnf4_gemv_nf4_grouped", "gnf4_gemv_mxfp4_grouped",
                             "gnf4_dgrad_nf4_grouped", "gnf4_dgrad_mxfp4_grouped"):
                    fn = getattr(lib, name)
                    fn.restype = ctypes.c_int
                    fn.argtypes = [_P, _P, _P, _P, _P, ctypes.c_int, _I64, _I64,
                                   _P, ctypes.c_int]
                # 13 arguments: the int64 trio needs registered argtypes
                # (reference gnf4_native/build.py:121-129)
                lib.gnf4_gemv_nf4_ffn_grouped.restype = ctypes.c_int
                lib.gnf4_gemv_nf4_ffn_grouped.argtypes = [
                    _P, _P, _P, _P, _P, _P, _P, ctypes.c_int, _I64, _I64, _I64, _P,
                    ctypes.c_int]
                lib.gnf4_route_epilogue_bf16.restype = None
                lib.gnf4_route_epilogue_bf16.argtypes = [
                    _P, _I64, _I64, _I64, ctypes.c_int, ctypes.c_int, _P, _I64, _P, _I64]
                _ref, _ref_path = lib, path
                break
    return _ref


def ref_path():
    ref_lib()
    return _ref_path


def _prep(a, packed, scales, sizes, expert_ids, fmt):
    a = np.ascontiguousarray(a, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(
        scales, dtype=np.float32 if fmt == "nf4" else np.uint8)
    eids = np.ascontiguousarray(np.asarray(expert_ids, dtype=np.int64))
    sz = np.ascontiguousarray(np.asarray(sizes, dtype=np.int32))
    return a, packed, scales, eids, sz


def gemv_grouped(a, packed, scales, sizes, expert_ids, *, fmt, threads=0):
    """Oracle forward (fp32 [R, N]), locked tree."""
    a, packed, scales, eids, sz = _prep(a, packed, scales, sizes, expert_ids, fmt)
    E, N, half = packed.shape
    out = np.empty((a.shape[0], N), dtype=np.float32)
    rc = oracle_lib().gnf4o_gemv_grouped(
        FMT[fmt], _ptr(a), _ptr(packed), _ptr(scales), _ptr(eids), _ptr(sz),
        len(sz), E, N, half * 2, _ptr(out), threads)
    if rc:
        raise ValueError(f"gnf4o_gemv_grouped rejected the call (rc={rc})")
    return out


def dgrad_grouped(g, packed, scales, sizes, expert_ids, *, fmt, threads=0):
    """Oracle dgrad (fp32 [R, K]), ascending-n chain."""
    g, packed, scales, eids, sz = _prep(g, packed, scales, sizes, expert_ids, fmt)
    E, N, half = packed.shape
    out = np.zeros((g.shape[0], half * 2), dtype=np.float32)
    rc = oracle_lib().gnf4o_dgrad_grouped(
        FMT[fmt], _ptr(g), _ptr(packed), _ptr(scales), _ptr(eids), _ptr(sz),
        len(sz), E, N, half * 2, _ptr(out), threads)
    if rc:
        raise ValueError(f"gnf4o_dgrad_grouped rejected the call (rc={rc})")
    return out


def ref_gemv_grouped(a, packed, scales, sizes, expert_ids, *, fmt, threads=0):
    """The compiled reference's forward (sizes must be >= 1, G <= 512)."""
    lib = ref_lib()
    if lib is None:
        raise RuntimeError("reference build absent (oracle/_ref)")
    a, packed, scales, eids, sz = _prep(a, packed, scales, sizes, expert_ids, fmt)
    E, N, half = packed.shape
    out = np.empty((a.shape[0], N), dtype=np.float32)
    fn = lib.gnf4_gemv_nf4_grouped if fmt == "nf4" else lib.gnf4_gemv_mxfp4_grouped
    rc = fn(_ptr(a), _ptr(packed), _ptr(scales), _ptr(eids), _ptr(sz), len(sz),
            N, half * 2, _ptr(out), threads)
    if rc:
        raise ValueError(f"reference gemv rejected the call (rc={rc})")
    return out


def ref_dgrad_grouped(g, packed, scales, sizes, expert_ids, *, fmt, threads=0):
    """The compiled reference's dgrad (caller-zeroed output)."""
    lib = ref_lib()
    if lib is None:
        raise RuntimeError("reference build absent (oracle/_ref)")
    g, packed, scales, eids, sz = _prep(g, packed, scales, sizes, expert_ids, fmt)
    E, N, half = packed.shape
    out = np.zeros((g.shape[0], half * 2), dtype=np.float32)
    fn = lib.gnf4_dgrad_nf4_grouped if fmt == "nf4" else lib.gnf4_dgrad_mxfp4_grouped
    rc = fn(_ptr(g), _ptr(packed), _ptr(scales), _ptr(eids), _ptr(sz), len(sz),
            N, half * 2, _ptr(out), threads)
    if rc:
        raise ValueError(f"reference dgrad rejected the call (rc={rc})")
    return out


def silu_locked(x):
    """The locked fp32 silu (C oracle), elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    oracle_lib().gnf4o_silu_locked(_ptr(x), _ptr(out), x.size)
    return out


def _prep_ffn(a, gu_p, gu_a, dn_p, dn_a, sizes, expert_ids):
    a = np.ascontiguousarray(a, dtype=np.float32)
    gu_p, dn_p = (np.ascontiguousarray(t, dtype=np.uint8) for t in (gu_p, dn_p))
    gu_a, dn_a = (np.ascontiguousarray(t, dtype=np.float32) for t in (gu_a, dn_a))
    eids = np.ascontiguousarray(np.asarray(expert_ids, dtype=np.int64))
    sz = np.ascontiguousarray(np.asarray(sizes, dtype=np.int32))
    return a, gu_p, gu_a, dn_p, dn_a, eids, sz


def ffn_grouped(a, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes, expert_ids, *,
                threads=0):
    """Oracle fused NF4 FFN: gemv -> silu_locked(gate) * up -> gemv, fp32."""
    a, gu_p, gu_a, dn_p, dn_a, eids, sz = _prep_ffn(a, gu_packed, gu_absmax, dn_packed,
                                                    dn_absmax, sizes, expert_ids)
    E, n_gu, half = gu_p.shape
    n_dn = dn_p.shape[1]
    out = np.empty((a.shape[0], n_dn), dtype=np.float32)
    rc = oracle_lib().gnf4o_ffn_grouped(
        _ptr(a), _ptr(gu_p), _ptr(gu_a), _ptr(dn_p), _ptr(dn_a), _ptr(eids), _ptr(sz),
        len(sz), E, n_gu, half * 2, n_dn, _ptr(out), threads)
    if rc:
        raise ValueError(f"gnf4o_ffn_grouped rejected the call (rc={rc})")
    return out


def ref_ffn_grouped(a, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes, expert_ids, *,
                    threads=0):
    """The compiled reference's fused FFN (sizes >= 1, G <= 512)."""
    lib = ref_lib()
    if lib is None:
        raise RuntimeError("reference build absent (oracle/_ref)")
    a, gu_p, gu_a, dn_p, dn_a, eids, sz = _prep_ffn(a, gu_packed, gu_absmax, dn_packed,
                                                    dn_absmax, sizes, expert_ids)
    n_gu, half = gu_p.shape[1], gu_p.shape[2]
    n_dn = dn_p.shape[1]
    out = np.empty((a.shape[0], n_dn), dtype=np.float32)
    rc = lib.gnf4_gemv_nf4_ffn_grouped(
        _ptr(a), _ptr(gu_p), _ptr(gu_a), _ptr(dn_p), _ptr(dn_a), _ptr(eids), _ptr(sz),
        len(sz), n_gu, half * 2, n_dn, _ptr(out), threads)
    if rc:
        raise ValueError(f"reference ffn rejected the call (rc={rc})")
    return out


def route_topk(logits, k, mode, norm):
    """Oracle top-k + softmax weights: (idx int64 [T, k], wts uint16 bf16 bits)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    idx = np.zeros((T, k), dtype=np.int64)
    wts = np.zeros((T, k), dtype=np.uint16)
    rc = oracle_lib().gnf4o_route_topk(_ptr(lg), T, E, k, mode, int(norm), _ptr(idx), _ptr(wts))
    if rc:
        raise ValueError(f"gnf4o_route_topk rejected the call (rc={rc})")
    return idx, wts


def ref_route_topk(logits, k, mode, norm):
    """The compiled reference's gnf4_route_epilogue_bf16."""
    lib = ref_lib()
    if lib is None:
        raise RuntimeError("reference build absent (oracle/_ref)")
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    idx = np.zeros((T, k), dtype=np.int64)
    wts = np.zeros((T, k), dtype=np.uint16)
    lib.gnf4_route_epilogue_bf16(_ptr(lg), T, E, k, mode, int(norm), _ptr(idx), k, _ptr(wts), k)
    return idx, wts


def route_groups(topk_ids, E):
    """Oracle grouping of the flattened routed rows: (eids, row_off, order,
    pos) as int32 arrays, eids / row_off over the active groups only."""
    ids = np.ascontiguousarray(np.asarray(topk_ids, dtype=np.int64).reshape(-1))
    N = ids.size
    eids = np.zeros(max(E, 1), dtype=np.int32)
    row_off = np.zeros(max(E, 1) + 1, dtype=np.int32)
    order = np.zeros(max(N, 1), dtype=np.int32)
    pos = np.zeros(max(N, 1), dtype=np.int32)
    g = oracle_lib().gnf4o_route_groups(_ptr(ids), N, E, _ptr(eids), _ptr(row_off),
                                        _ptr(order), _ptr(pos))
    if g < 0:
        raise ValueError(f"gnf4o_route_groups rejected the call (rc={g})")
    return eids[:g], row_off[:g + 1], order[:N], pos[:N]


def oracle_luts():
    lib = oracle_lib()
    nf4 = np.ctypeslib.as_array(lib.gnf4o_nf4_lut(), shape=(16,)).copy()
    fp4 = np.ctypeslib.as_array(lib.gnf4o_fp4_lut(), shape=(16,)).copy()
    return nf4, fp4


def build() -> None:
    """Compile the oracle (and the reference when its source is present)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True,
                   env=dict(os.environ))
