"""The C-ABI library loads on a GPU-less host, exports every symbol that
include/gnf4_hip.h declares, and rejects contract violations with -1 before
touching the device (no compute is launched here)."""
import ctypes
import re
from pathlib import Path

import pytest

import _hiplib

HEADER = Path(__file__).resolve().parents[1] / "include" / "gnf4_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|int64_t)\s+(gnf4_hip_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_expected_entry_points():
    names = set(declared_functions())
    assert {"gnf4_hip_nf4_fwd", "gnf4_hip_mxfp4_fwd", "gnf4_hip_nf4_dgrad",
            "gnf4_hip_mxfp4_dgrad", "gnf4_hip_grouped_fwd", "gnf4_hip_grouped_dgrad",
            "gnf4_hip_activations_to_bf16"} <= names


def test_library_exports_every_declared_symbol():
    lib = _hiplib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _hiplib.SIGNATURES, f"{name} has no registered ctypes signature"
    assert lib.gnf4_hip_abi_version() == _hiplib.ABI_VERSION


def test_signature_arity_matches_the_header():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name in declared_functions():
        m = re.search(name + r"\s*\((.*?)\)\s*;", text, flags=re.S)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(_hiplib.SIGNATURES[name]), name


def _fwd(lib, **over):
    args = dict(fmt=0, a=8, a_dtype=0, lda=64, B=16, sbe=1024, sbn=32, S=32, sse=32, ssn=1,
                eids=64, row_off=None, G=1, t0=None, tr=None, tg=None, nmt=0, bm=0,
                N=32, K=64, out=128, ldo=32, stream=None)
    args.update(over)
    return lib.gnf4_hip_grouped_fwd(*args.values())


def test_contract_violations_return_minus_one_without_a_device():
    lib = _hiplib.load()
    assert _fwd(lib, K=96) == -1            # NF4 needs K % 64 == 0
    assert _fwd(lib, fmt=1, K=48) == -1     # MXFP4 needs K % 32 == 0
    assert _fwd(lib, fmt=7) == -1
    assert _fwd(lib, a_dtype=1) == -1       # fp16 is widened first; the forward takes bf16
    assert _fwd(lib, sbn=24) == -1          # weight rows must be 16-byte aligned
    assert _fwd(lib, lda=60) == -1
    assert _fwd(lib, a=None) == -1
    assert _fwd(lib, nmt=2, t0=None) == -1  # tiled path needs the tile table
    assert lib.gnf4_hip_grouped_dgrad(0, 16, 0, 32, 16, 1024, 32, 32, 32, 1, 64, None, None,
                                      None, 1, 32, 32, 96, 128, 96, None) == -1
    assert lib.gnf4_hip_nf4_dgrad(16, 0, 32, 16, 1024, 32, 32, 32, 1, 64, 48, 48, 48, 0,
                                  32, 32, 64, 128, 64, None) == 0     # nothing to do


def test_widening_rejects_bad_arguments_without_a_device():
    lib = _hiplib.load()
    w = lib.gnf4_hip_activations_to_bf16
    assert w(16, _hiplib.DTYPE_BF16, 2, 64, 64, 16, 64, None) == -1   # bf16 needs no widening
    assert w(16, 9, 2, 64, 64, 16, 64, None) == -1
    assert w(16, _hiplib.DTYPE_F16, 2, 60, 64, 16, 64, None) == -1    # cols % 8
    assert w(16, _hiplib.DTYPE_F16, 2, 64, 60, 16, 64, None) == -1    # ld_src < cols
    assert w(16, _hiplib.DTYPE_F32, 2, 64, 68, 16, 64, None) == -1    # ld_src % 8
    assert w(8, _hiplib.DTYPE_F32, 2, 64, 64, 16, 64, None) == -1     # 16-byte alignment
    assert w(None, _hiplib.DTYPE_F32, 2, 64, 64, 16, 64, None) == -1
    assert w(None, _hiplib.DTYPE_F16, 0, 64, 64, None, 64, None) == 0  # nothing to do


def test_ffn_sync_size_is_the_flag_count_plus_header():
    lib = _hiplib.load()
    words = lib.gnf4_hip_ffn_sync_words
    # Qwen3 shapes, batch 1: 8 groups x 64 down units x 48 gate/up units
    assert words(8, 1536, 2048) == 16 + 8 * 64 * 48
    assert words(0, 1536, 2048) == 16
    assert words(3, 128, 24) == 16 + 3 * 1 * 4
    assert words(-1, 128, 24) == -1
