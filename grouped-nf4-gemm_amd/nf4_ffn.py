"""Grouped NF4 expert FFN on MI355X: gate_up -> silu(gate) * up -> down.

``gemm_nf4_ffn_grouped`` is the GPU form of the reference's fused CPU FFN
(``gemm_nf4_ffn_grouped_cpu``, kernel/cpu_grouped.py:288-346; C entry
gnf4_native/cpu_kernels.c:948-986), which the reference has only for its CPU
tier. Layouts and error behaviour follow that wrapper:
``gu_packed [E, 2H, K/2]`` u8 + ``gu_absmax [E, 2H, K/64]`` f32 (gate = the
first H outputs, up = the last H), ``dn_packed [E, N_dn, H/2]`` u8 +
``dn_absmax [E, N_dn, H/64]`` f32, ``H % 64 == 0``.

Two paths, both HIP:
  * every group at most 16 rows (decode): ONE launch of the fused kernel.
    gate/up units write the intermediate h straight from their epilogue and
    set per-call flags for the down units of their group; down units stream
    their weights meanwhile and start the moment their group's h is
    complete. No gu tensor is written, and there is no second or third
    launch. A down unit that never sees its flags (not expected) writes NaN
    into its output rows and sets a sticky error word
    (``ffn_sync_error()``).
  * larger groups: the tiled forward kernel for gate_up, the silu-multiply
    kernel, the tiled forward kernel for down.

Numerics: gate and up are the bf16 outputs of the forward kernel, h is
``bf16(silu_locked(gate) * up)`` with the reference's locked fp32 silu
(kernel/cpu_grouped.py:147-179), and the result is bf16. The fused call
gives the same bits as the three-launch composition, which is how the tests
pin it. For one-row groups the fused call is two launches (the gate_up GEMV
with the silu-multiply in its epilogue, then the down GEMV); larger groups
run one launch whose down units wait on flags set by the gate/up units. Against the reference's fp32 CPU FFN the bound is the tolerance
contract (docs/TOLERANCE_CONTRACT.md), like the forward op.
"""
from __future__ import annotations

import threading

import numpy as np

import torch

import _hiplib
import nf4_grouped
from nf4_grouped import (BLOCKSIZE, DECODE_MAX_ROWS, _aligned_rows, _bf16_activations,
                         _check_host_ids, _eids_device, _require_gpu, _scales_view,
                         _stream_ptr)

# Auto path choice: the fused launch saves the silu launch and a kernel
# boundary, and pays a device-scope hand-off per unit (h stores must complete
# before the flags go out, and down units hold their slot while they wait).
# Measured on MI355X at Qwen3-30B-A3B shapes (per layer, HIP graph, 112
# units per group): batch 1 (896 units) 13.7 us fused vs 15.3 us three-launch,
# batch 2 23.1 vs 22.8, batch 4 48.5 vs 35.3 -- once the batched decode
# kernels stream well, down units spinning in their slots cost more than the
# saved launch. The fused launch wins up to about 1000 workgroup units. (At
# batch 1 the fused call is now the two-launch GEMV form: 10.3 us per layer
# against 12.6 us for three launches.)
FUSED_MAX_UNITS = 1024


def _fused_units(G: int, H: int, n_dn: int) -> int:
    return G * (H // 16 + (n_dn + 31) // 32)


#: Largest group of the multi-row decode GEMV (the library's kGemvMaxRows
#: and kGemvMaxRowsNarrow): groups of up to 4 rows at 1024 < K <= 2048, up
#: to 2 rows at K <= 1024, run as one-row passes of the GEMV.
GEMV_MAX_ROWS = 4
GEMV_MAX_ROWS_NARROW = 2


def _gemv_stage(max_m: int, K: int) -> bool:
    """Whether a decode launch of this largest group and K takes the GEMV
    class (one-row groups always; multi-row ones as the library decides)."""
    if max_m == 1:
        return True
    if K % 64 or K > 2048:
        return False
    return max_m <= (GEMV_MAX_ROWS if K > 1024 else GEMV_MAX_ROWS_NARROW)


def _auto_fused(G: int, max_m: int, K: int, H: int, n_dn: int) -> bool:
    """The fused call where it measures faster: always when its gate_up
    stage is a GEMV (two launches, the silu-multiply in the first one's
    epilogue), else while the single launch has at most FUSED_MAX_UNITS
    units."""
    if max_m > DECODE_MAX_ROWS:
        return False
    return _gemv_stage(max_m, K) or _fused_units(G, H, n_dn) <= FUSED_MAX_UNITS


_SYNC_LOCK = threading.Lock()
_SYNC = {}      # (device index, stream handle) -> current int32 sync words
_RETIRED = []   # outgrown sync buffers: never freed (a captured graph may use them)


def _sync_words(dev, G: int, n_gu: int, n_dn: int):
    """The fused kernel's sync words for this device and stream. They start
    at zero and every call leaves its flags at zero, so one buffer serves
    every stream-ordered call; a separate buffer per stream keeps concurrent
    streams apart. A call that needs more words gets a larger buffer; the
    old one is kept alive for the life of the process, because a graph
    captured earlier still holds its address (graph captures share one
    capture stream, hence one key)."""
    key = (dev.index, _stream_ptr(dev))
    need = int(_hiplib.load().gnf4_hip_ffn_sync_words(G, n_gu, n_dn))
    with _SYNC_LOCK:
        buf = _SYNC.get(key)
        if buf is None or buf.numel() < need:
            if buf is not None:
                _RETIRED.append(buf)
            buf = torch.zeros(max(need, 4096), dtype=torch.int32, device=dev)
            _SYNC[key] = buf
    return buf


def _device_buffers(device):
    dev = torch.device(device if device is not None else "cuda")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    with _SYNC_LOCK:
        return ([b for (d, _s), b in _SYNC.items() if d == idx]
                + [b for b in _RETIRED if b.device.index == idx])


def ffn_sync_error(device=None) -> bool:
    """True if a down unit of any fused call on this device gave up waiting
    for its h since the last ``ffn_sync_clear`` (that call's affected output
    rows are NaN). Reads device memory: it synchronises, so it is meant for
    tests and diagnostics."""
    return any(int(b[0].item()) != 0 for b in _device_buffers(device))


def ffn_sync_clear(device=None) -> None:
    """Zero every sync buffer of this device (error word and flags): after
    an error, graph replays of fused calls are valid again only after this.
    Stream-ordered on the current stream; no fused call may be in flight on
    another stream."""
    for b in _device_buffers(device):
        b.zero_()


def set_spin_limit(polls: int) -> None:
    """Polls a down unit of later fused launches makes before it gives up
    (default 2**22). For diagnostics and tests of the time-out path."""
    _hiplib.check(_hiplib.load().gnf4_hip_ffn_set_spin_limit(int(polls)), "set_spin_limit")


def silu_mul_locked(gu: torch.Tensor) -> torch.Tensor:
    """``h = bf16(silu_locked(gu[:, :H]) * gu[:, H:])`` for bf16 ``gu [T, 2H]``
    (one HIP launch). The activation of the fused FFN, unfused."""
    _require_gpu(gu, "silu_mul_locked",
                 "The CPU form is silu_locked_ref in the reference's cpu_grouped.")
    if gu.dtype != torch.bfloat16:
        raise TypeError(f"silu_mul_locked: gu must be bfloat16, got {gu.dtype}")
    T, n2 = gu.shape
    if n2 % 2 or (n2 // 2) % 8:
        raise ValueError(f"gu width {n2} must be 2H with H % 8 == 0")
    H = n2 // 2
    if gu.stride(-1) != 1 or gu.stride(0) % 8 or gu.data_ptr() % 16:
        gu = gu.contiguous()
    h = torch.empty(T, H, dtype=torch.bfloat16, device=gu.device)
    with torch.cuda.device(gu.device):
        rc = _hiplib.load().gnf4_hip_silu_mul(gu.data_ptr(), gu.stride(0), T, H, h.data_ptr(),
                                              h.stride(0), _stream_ptr(gu.device))
    _hiplib.check(rc, "silu_mul_locked")
    return h


def _check(a_cat, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes, expert_ids):
    """The reference wrapper's checks (kernel/cpu_grouped.py:306-331)."""
    T = a_cat.shape[0]
    assert sum(int(m) for m in sizes) == T, (sum(int(m) for m in sizes), T)
    if len(sizes) != len(expert_ids):
        raise ValueError(f"{len(sizes)} group sizes but {len(expert_ids)} expert ids")
    return _check_shapes(a_cat, gu_packed, gu_absmax, dn_packed, dn_absmax)


def _check_shapes(a_cat, gu_packed, gu_absmax, dn_packed, dn_absmax):
    T, K = a_cat.shape
    if gu_packed.dtype != torch.uint8 or dn_packed.dtype != torch.uint8:
        raise TypeError("packed weights must be uint8")
    if gu_absmax.dtype != torch.float32 or dn_absmax.dtype != torch.float32:
        raise TypeError("absmax must be fp32")
    n_gu = gu_packed.shape[1]
    if n_gu % 2:
        raise ValueError(f"gu output width {n_gu} must be even (gate/up halves)")
    h_dim = n_gu // 2
    if K % BLOCKSIZE or gu_packed.shape[2] * 2 != K:
        raise ValueError("K mismatch or K % 64 != 0")
    if h_dim % BLOCKSIZE or dn_packed.shape[2] * 2 != h_dim:
        raise ValueError(f"dn expects K={h_dim} (=H) with H % 64 == 0, "
                         f"got packed K={dn_packed.shape[2] * 2}")
    if dn_packed.shape[0] != gu_packed.shape[0]:
        raise ValueError("gu/dn expert counts differ")
    E, n_dn = gu_packed.shape[0], dn_packed.shape[1]
    if tuple(gu_absmax.shape) != (E, n_gu, K // BLOCKSIZE):
        raise ValueError(f"gu_absmax shape {tuple(gu_absmax.shape)} != {(E, n_gu, K // 64)}")
    if tuple(dn_absmax.shape) != (E, n_dn, h_dim // BLOCKSIZE):
        raise ValueError(f"dn_absmax shape {tuple(dn_absmax.shape)} != "
                         f"{(E, n_dn, h_dim // 64)}")
    dev = a_cat.device
    if any(t.device != dev for t in (gu_packed, gu_absmax, dn_packed, dn_absmax)):
        raise ValueError("activations and weights must be on the same device")
    return T, K, h_dim, n_dn


def gemm_nf4_ffn_grouped(a_cat, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes,
                         expert_ids, fused: bool | None = None):
    """Grouped NF4 expert FFN ``dn(silu(gate) * up)`` on the GPU.

    ``a_cat [T, K]`` bf16 (fp16 / fp32 are rounded to bf16 first), rows sorted
    by group; ``sizes`` per-group row counts (zero-size groups allowed);
    ``expert_ids [G]`` list, CPU tensor or device tensor. Returns ``[T, N_dn]``
    bf16. ``fused``: None picks the fused call when every group has at
    most 16 rows and either its gate_up stage is a GEMV (``_gemv_stage``:
    groups of at most 4 rows at 1024 < K <= 2048, 2 at K <= 1024) or the
    single launch has at most
    ``FUSED_MAX_UNITS`` workgroup units (where it measures faster); False
    forces the three-launch
    composition; True requires the fused launch. Both give the same bits."""
    _require_gpu(a_cat, "gemm_nf4_ffn_grouped",
                 "The CPU form is the reference's gemm_nf4_ffn_grouped_cpu; a "
                 "checkable decode of the weights is dequant_ref(packed, absmax, N, K).")
    T, K, H, n_dn = _check(a_cat, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes,
                           expert_ids)
    dev = a_cat.device
    E = gu_packed.shape[0]
    sizes_i = [int(m) for m in sizes]
    G = len(sizes_i)
    max_m = max(sizes_i, default=0)
    if fused is None:
        fused = _auto_fused(G, max_m, K, H, n_dn)
    elif fused and max_m > DECODE_MAX_ROWS:
        raise ValueError(f"the fused FFN launch takes groups of at most {DECODE_MAX_ROWS} "
                         f"rows, got {max_m}")
    if T == 0 or G == 0:
        return torch.zeros(T, n_dn, dtype=torch.bfloat16, device=dev)
    eids_dev = _eids_device(expert_ids, dev)
    if eids_dev is None:
        _check_host_ids(expert_ids, E)
    if not fused:
        gu = nf4_grouped.gemm_4bit_grouped(a_cat, gu_packed, gu_absmax, sizes, expert_ids)
        h = silu_mul_locked(gu)
        return nf4_grouped.gemm_4bit_grouped(h, dn_packed, dn_absmax, sizes, expert_ids)
    a = _bf16_activations(a_cat, "gemm_nf4_ffn_grouped")
    if eids_dev is None and G <= nf4_grouped.IDS_ARG_MAX:
        ro = None
        if not (min(sizes_i) == 1 and max_m == 1):
            ro = np.zeros(G + 1, dtype=np.int32)
            np.cumsum(np.asarray(sizes_i, dtype=np.int32), out=ro[1:])
        out = _launch_fused_ids(a, gu_packed, gu_absmax, dn_packed, dn_absmax,
                                nf4_grouped._np_ids(expert_ids), ro, G, max_m)
        if out is not None:
            return out
    row_off = [0]
    for m in sizes_i:
        row_off.append(row_off[-1] + m)
    host_eids = [] if eids_dev is not None else expert_ids
    (e_p, r_p), keep = nf4_grouped._upload_tables((host_eids, row_off), dev,
                                                  torch.cuda.current_stream(dev), host_ok=True)
    eids = eids_dev.data_ptr() if eids_dev is not None else e_p
    out = _launch_fused(a, gu_packed, gu_absmax, dn_packed, dn_absmax, eids, r_p, G, max_m)
    del keep, eids_dev   # the index tensors stay alive until the launch is enqueued
    return out


def _launch_fused(a, gu_packed, gu_absmax, dn_packed, dn_absmax, eids, row_off, G: int,
                  max_m: int, h=None, out=None, op="gemm_nf4_ffn_grouped"):
    """The fused kernel over device group tables (``eids [G]`` and
    ``row_off [G + 1]`` int32, as tensors or device addresses; ``max_m`` an
    upper bound of the largest group, <= 16). ``a`` bf16 [T, K]."""
    T, K = a.shape
    H, n_dn = gu_packed.shape[1] // 2, dn_packed.shape[1]
    dev = a.device
    Wg, Sg = _aligned_rows(gu_packed, 16), _scales_view(gu_absmax)
    Wd, Sd = _aligned_rows(dn_packed, 16), _scales_view(dn_absmax)
    if h is None:
        h = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    if out is None:
        out = torch.empty(T, n_dn, dtype=torch.bfloat16, device=dev)
    sync = _sync_words(dev, G, 2 * H, n_dn)
    with torch.cuda.device(dev):
        rc = _hiplib.load().gnf4_hip_nf4_ffn_fwd(
            a.data_ptr(), _hiplib.DTYPE_BF16, a.stride(0),
            Wg.data_ptr(), Wg.stride(0), Wg.stride(1), Sg.data_ptr(), Sg.stride(0), Sg.stride(1),
            Wd.data_ptr(), Wd.stride(0), Wd.stride(1), Sd.data_ptr(), Sd.stride(0), Sd.stride(1),
            eids if isinstance(eids, int) else eids.data_ptr(),
            row_off if isinstance(row_off, int) else row_off.data_ptr(), G, max(max_m, 1),
            2 * H, K, n_dn,
            h.data_ptr(), h.stride(0), sync.data_ptr(), sync.numel(),
            out.data_ptr(), out.stride(0), _stream_ptr(dev))
    _hiplib.check(rc, op)
    return out


def _launch_fused_ids(a, gu_packed, gu_absmax, dn_packed, dn_absmax, ids32, row_off, G: int,
                      max_m: int, h=None, out=None, op="gemm_nf4_ffn_grouped"):
    """The fused FFN with host group tables (``ids32 [G]``, ``row_off
    [G + 1]`` or None for one row per group, int32 numpy) passed in the
    kernels' arguments (``gnf4_hip_nf4_ffn_decode_ids``): no upload and no
    table read ahead of the weights. None when the library leaves the call to
    the device-table entry (a stage that is not a GEMV launch, or G above its
    table size)."""
    T, K = a.shape
    H, n_dn = gu_packed.shape[1] // 2, dn_packed.shape[1]
    dev = a.device
    Wg, Sg = _aligned_rows(gu_packed, 16), _scales_view(gu_absmax)
    Wd, Sd = _aligned_rows(dn_packed, 16), _scales_view(dn_absmax)
    if h is None:
        h = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    if out is None:
        out = torch.empty(T, n_dn, dtype=torch.bfloat16, device=dev)
    with nf4_grouped._device_ctx(dev):
        rc = _hiplib.load().gnf4_hip_nf4_ffn_decode_ids(
            a.data_ptr(), _hiplib.DTYPE_BF16, a.stride(0),
            Wg.data_ptr(), Wg.stride(0), Wg.stride(1), Sg.data_ptr(), Sg.stride(0), Sg.stride(1),
            Wd.data_ptr(), Wd.stride(0), Wd.stride(1), Sd.data_ptr(), Sd.stride(0), Sd.stride(1),
            ids32.ctypes.data, row_off.ctypes.data if row_off is not None else None, G,
            max(max_m, 1), 2 * H, K, n_dn, h.data_ptr(), h.stride(0),
            out.data_ptr(), out.stride(0), _stream_ptr(dev))
    if rc == 1:
        return None
    _hiplib.check(rc, op)
    return out


def launch_ffn_planned(a_cat, gu_packed, gu_absmax, dn_packed, dn_absmax, plan, h=None,
                       out=None):
    """Fused FFN launch with a prepared decode ``nf4_grouped.GroupPlan``: the
    kernel and nothing else (no table upload), for graph capture and timing
    loops. ``a_cat`` bf16; ``h`` / ``out`` optional preallocated workspace
    and result."""
    if not plan.decode:
        raise ValueError("launch_ffn_planned needs a decode plan (every group <= 16 rows)")
    T, K, H, n_dn = _check_shapes(a_cat, gu_packed, gu_absmax, dn_packed, dn_absmax)
    E = gu_packed.shape[0]
    if plan.min_id < 0 or plan.max_id >= E:
        raise ValueError(f"expert id out of range [0, {E})")
    a = _bf16_activations(a_cat, "launch_ffn_planned")
    if 0 < plan.G <= nf4_grouped.IDS_ARG_MAX:
        res = _launch_fused_ids(a, gu_packed, gu_absmax, dn_packed, dn_absmax, plan.host_ids,
                                plan.host_row_off, plan.G, plan.max_m, h=h, out=out,
                                op="launch_ffn_planned")
        if res is not None:
            return res
    return _launch_fused(a, gu_packed, gu_absmax, dn_packed, dn_absmax, plan.eids, plan.row_off,
                         plan.G, plan.max_m, h=h, out=out, op="launch_ffn_planned")

