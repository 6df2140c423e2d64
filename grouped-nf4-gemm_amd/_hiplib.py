"""ctypes binding of libgnf4_hip.so (the C ABI in include/gnf4_hip.h).

The library is loaded from this directory; there is no fallback. A missing or
stale build raises with the command that fixes it. All int64 parameters carry
registered argtypes (the reference learned that the hard way,
gnf4_native/build.py:113-116).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libgnf4_hip.so"
ABI_VERSION = 14

FMT_NF4 = 0
FMT_MXFP4 = 1
DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64

# name -> argtypes; every entry point returns int
SIGNATURES = {
    "gnf4_hip_abi_version": [],
    "gnf4_hip_device_cus": [],
    "gnf4_hip_copy_to_device": [_P, _P, _I64, _P],
    "gnf4_hip_host_device_address": [_P, _P],
    "gnf4_hip_activations_to_bf16": [_P, _I, _I64, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_silu_mul": [_P, _I64, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_ffn_sync_words": [_I, _I64, _I64],
    "gnf4_hip_ffn_set_spin_limit": [_I],
    "gnf4_hip_nf4_ffn_fwd": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                             _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I, _I,
                             _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P],
    "gnf4_hip_nf4_ffn_decode_ids": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                    _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I, _I,
                                    _I64, _I64, _I64, _P, _I64, _P, _I64, _P],
    "gnf4_hip_nf4_ffn_noalloc_reset": [_P, _P],
    "gnf4_hip_nf4_ffn_fwd_noalloc": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                     _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I, _I,
                                     _I64, _I64, _I64, _P, _I64, _P, _I64, _P],
    "gnf4_hip_route_topk": [_P, _I64, _I64, _I64, _I, _I, _I, _P, _I64, _P, _I64, _P],
    "gnf4_hip_route_groups": [_P, _I64, _I64, _I, _I64, _I, _I, _P, _P, _P, _P, _P, _P],
    "gnf4_hip_route_decode": [_P, _I64, _I64, _I64, _I, _I, _I, _P, _I64, _P, _I64, _P, _I64,
                              _I64, _I, _I, _P, _P, _P, _P, _P, _P, _I64, _P],
    "gnf4_hip_gather_rows": [_P, _I64, _P, _I64, _I, _I64, _P, _I64, _P],
    "gnf4_hip_route_combine": [_P, _I64, _P, _P, _I64, _I64, _I, _I64, _P, _I64, _P],
    "gnf4_hip_grouped_fwd": [_I, _P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                             _P, _P, _I, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_grouped_decode_ids": [_I, _P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                    _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_grouped_decode_pairs": [_I, _P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                    _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_grouped_decode_routed": [_I, _P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                    _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_grouped_fwd_tiles": [_I, _P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                   _P, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_nf4_fwd": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                         _P, _P, _I, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_nf4_fwd_fp32w": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                               _P, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_mxfp4_fwd": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                           _P, _P, _I, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_grouped_dgrad": [_I, _P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                               _P, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_grouped_dgrad_tiles": [_I, _P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                     _P, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_nf4_dgrad": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                           _P, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
    "gnf4_hip_mxfp4_dgrad": [_P, _I, _I64, _P, _I64, _I64, _P, _I64, _I64,
                             _P, _P, _P, _P, _I, _I, _I64, _I64, _P, _I64, _P],
}

# entry points that do not return int
RESTYPES = {"gnf4_hip_ffn_sync_words": ctypes.c_int64}

_lib = None


class HipLibraryError(RuntimeError):
    pass


def load():
    """The loaded library. Raises HipLibraryError when it is absent or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HipLibraryError(
            f"grouped-nf4 HIP library missing at {LIB_PATH}: build it with "
            f"`python {HERE / 'build.py'}` (hipcc, gfx950). There is no CPU "
            "or Triton fallback for this op.")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    ver = lib.gnf4_hip_abi_version()
    if ver != ABI_VERSION:
        raise HipLibraryError(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}: rebuild it")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc == -1:
        raise ValueError(f"{what}: the HIP library rejected the arguments "
                         "(shape, stride or alignment contract, rc=-1)")
    if rc != 0:
        raise RuntimeError(f"{what}: kernel launch failed (rc={rc})")
