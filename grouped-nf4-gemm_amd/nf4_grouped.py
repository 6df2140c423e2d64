"""Grouped W4A16 GEMM over NF4 expert stacks on MI355X (gfx950), dequant fused.

Drop-in for the reference module of the same name (kernel/nf4_grouped.py):
same entry points, keyword arguments, exported helpers and error behaviour.

``gemm_4bit_grouped`` computes, in one launch for all active experts,
``out[t, :] = a[t, :] @ dequant_nf4(B[e(t)]).T`` for tokens grouped by expert;
``dgrad_4bit_grouped`` is its backward with respect to the activations. The
packed ``[E, N, K/2]`` bytes are decoded inside the kernel and never written
back to memory. Both call hand-written HIP kernels (``csrc/gnf4_hip.hip``)
through the C ABI in ``include/gnf4_hip.h``; there is no CPU, Triton or
eager-PyTorch fallback. On a non-GPU tensor the ops raise.

Numerics. Decode (every group of at most 16 rows) keeps the codebook in
fp32, as the reference's GEMV does (kernel/nf4_grouped.py:508-511): each
64-element block's dot product of fp32 codebook values and bf16 activations
is formed in fp32 and scaled by absmax once, in fp32. One-row groups use
fp32 FMAs; larger groups put an exact three-part bf16 split of the codebook
through three bf16 MFMAs. The tiled kernels (larger groups) use bf16 weights
``bf16(fp32(NF4[code] * absmax))`` -- the same values ``dequant_ref(...)``
gives after ``.to(bfloat16)``, the reference's opt-in VARIANT 3
(kernel/nf4_grouped.py:438-445) -- into bf16 MFMA with fp32 accumulation.
Every output is rounded to bf16 once. fp16 and fp32 activations are first
rounded to bf16 (nearest-even), so their result equals the forward of
``a.to(bfloat16)`` bit for bit. The stated bound is the tolerance contract
(reference docs/TOLERANCE_CONTRACT.md): B-rel <= 2x the bf16
dequant-then-matmul path against an fp64 reference, <= 1e-2, and the
fidelity ordering P-fid (decode strictly below the dequant path's error,
tiles tied with it).
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import numpy as np
import threading

import torch

import _hiplib

# The NF4 codebook (reference kernel/nf4_grouped.py:53-70). Code 7 is exactly 0.
NF4_LUT = [
    -1.0,
    -0.6961928009986877,
    -0.5250730514526367,
    -0.39491748809814453,
    -0.28444138169288635,
    -0.18477343022823334,
    -0.09105003625154495,
    0.0,
    0.07958029955625534,
    0.16093020141124725,
    0.24611230194568634,
    0.33791524171829224,
    0.44070982933044434,
    0.5626170039176941,
    0.7229568362236023,
    1.0,
]
BLOCKSIZE = 64  # quant blocksize; K % 64 == 0 enforced

#: The reference gates its register-LUT mainloop on triton's ``tl.gather``.
#: This build has one mainloop (LDS pair table + bf16 MFMA); the flag stays
#: exported and True so callers that branch on it take the default path.
HAS_TL_GATHER = True

# Dispatch constants, kept with the reference's values and meaning
# (kernel/nf4_grouped.py:593-607): the byte floor below which a product
# integration should prefer the dequant path, and the per-split block floor
# of the split-K plan.
DECODE_MIN_FUSED_BYTES = 3_000_000
SPLITK_MIN_BLOCKS = 32

#: (BLOCK_M, BLOCK_N, BLOCK_K, num_warps) default of the dgrad launch
#: (reference kernel/nf4_grouped.py:1031). Here only BLOCK_M selects a tile
#: height; the contraction step is fixed, so no config changes output bits.
_DGRAD_DEFAULT = (32, 64, 64, 2)

#: Largest group the decode kernel takes (rows of one MFMA A tile).
DECODE_MAX_ROWS = 16


def repack_from_bnb(packed_list, states, N: int, K: int):
    """Per-expert bitsandbytes ``quantize_4bit`` results -> the stacked
    ``B [E, N, K/2]`` uint8 and ``absmax [E, N, K/64]`` fp32 this op takes
    (reference kernel/nf4_grouped.py:74-96). bitsandbytes keeps both flat and
    row-major, so with K % 64 == 0 each is a reshape; a nested
    (compress_statistics) state's absmax is first restored with
    bitsandbytes' own blockwise dequantize."""
    if K % BLOCKSIZE:
        raise AssertionError(f"K={K} is not a multiple of blocksize {BLOCKSIZE}")

    def absmax_of(state):
        if not getattr(state, "nested", False):
            return state.absmax
        from bitsandbytes import functional as bnb_f
        return bnb_f.dequantize_blockwise(state.absmax, state.state2) + state.offset

    B = torch.stack([p.reshape(N, K // 2) for p in packed_list])
    A = torch.stack([absmax_of(st).to(torch.float32).reshape(N, K // BLOCKSIZE)
                     for st in states])
    return B.contiguous(), A.contiguous()


# ------------------------------------------------------------------ indices --

class _PinnedIndexArena:
    """Pinned host staging for the small int32 index arrays, used while a
    stream is being captured into a graph (reference kernel/nf4_grouped.py:
    99-226). A pageable ``torch.tensor(list, device=...)`` synchronises, which
    a capture forbids; a copy from pinned memory that already exists does not.
    Slices taken under capture are owned forever -- replays re-read them -- so
    the bump pointer never rewinds, and the arena refuses to grow inside a
    capture. Size it with ``GNF4_PIN_ARENA_INTS`` or ``reserve()``."""

    DEFAULT_INTS = int(os.environ.get("GNF4_PIN_ARENA_INTS", 1 << 20))

    def __init__(self, device, n: int | None = None):
        self.device = device
        self.host = torch.empty(n or self.DEFAULT_INTS, dtype=torch.int32, pin_memory=True)
        self.off = 0
        self._retired: list = []

    @staticmethod
    def _capturing() -> bool:
        try:
            return torch.cuda.is_current_stream_capturing()
        except Exception:
            return False

    def take(self, n: int):
        capturing = self._capturing()
        if self.off + n > self.host.numel():
            if capturing:
                raise RuntimeError(
                    "grouped-nf4: the pinned index arena (%d int32, %d owned by "
                    "earlier captures) cannot hold %d more ints, and growing it "
                    "would allocate pinned memory inside the capture. Set "
                    "GNF4_PIN_ARENA_INTS to at least %d, or call reserve() "
                    "before capturing." % (self.host.numel(), self.off, n, 2 * (self.off + n)))
            self._grow(self.off + n)
        view = self.host[self.off:self.off + n]
        self.off += n
        return view, capturing

    def _grow(self, need: int):
        self._retired.append(self.host)       # live graphs may still read it
        fresh = torch.empty(max(2 * self.host.numel(), need), dtype=torch.int32,
                            pin_memory=True)
        fresh[: self.off] = self.host[: self.off]
        self.host = fresh

    def reserve(self, n_more: int):
        if self._capturing():
            raise RuntimeError("reserve() inside a capture would allocate pinned "
                               "memory in the region; call it before capturing.")
        if self.off + n_more > self.host.numel():
            self._grow(self.off + n_more)

    def mark(self):
        """Kept for call-site compatibility; nothing rewinds, nothing waits."""


class _PinnedRing:
    """Outside capture: a pinned staging ring per (device, stream), so an
    index upload is an asynchronous copy that never stalls the host on the
    GPU (the reference's pageable copy synchronises). The ring is cut into
    PARTS parts; an event is recorded on the stream when the ring leaves a
    part, and the host waits for that event before it writes into the part
    again (long done in practice). Values go in through a numpy view of the
    pinned memory (no temporary tensor)."""

    INTS = 1 << 16
    PARTS = 8

    def __init__(self):
        self.host = torch.empty(self.INTS, dtype=torch.int32, pin_memory=True)
        self.np = self.host.numpy()
        self.events = [None] * self.PARTS
        self.part = 0     # the part being filled
        self.off = 0      # next free int in it
        self.lock = threading.Lock()

    def stage(self, flat, dev, stream):
        n = len(flat)
        size = self.INTS // self.PARTS
        with self.lock:
            if n > size:
                # larger than a part (not on any launch path's shapes): a
                # pinned buffer of its own, kept until its copy has run
                host = torch.empty(n, dtype=torch.int32, pin_memory=True)
                host.numpy()[:] = flat
                out = host.to(dev, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(stream)
                ev.synchronize()
                return out
            if self.off + n > size:
                ev = self.events[self.part]
                if ev is None:
                    ev = self.events[self.part] = torch.cuda.Event()
                ev.record(stream)                      # after this part's copies
                self.part = (self.part + 1) % self.PARTS
                self.off = 0
                nxt = self.events[self.part]
                if nxt is not None:
                    nxt.synchronize()                  # its last round's copies ran
            base = self.part * size + self.off
            self.np[base:base + n] = flat
            out = self.host[base:base + n].to(dev, non_blocking=True)
            self.off += n
            return out


class _TableRing:
    """Outside capture, the launch paths' group tables (expert ids, row
    offsets, tile table) per (device, stream): a pinned host ring and a
    device ring of the same size. A call writes its ints into the host ring
    through a numpy view; no tensor is made per call. Decode launches
    (``host_ok``: each workgroup reads its group's three words once) read
    them there, at the ring's device address, with no copy; tile launches,
    which read their tile table once per tile, get one stream-ordered copy
    into the device ring. Both rings are cut into PARTS parts; an event
    recorded on the stream when the ring leaves a part guards both sides of
    that part (its copies, and every kernel enqueued before the event, have
    run when it completes), and the host waits for it before writing into
    the part again (long done in practice)."""

    INTS = 1 << 16
    PARTS = 8

    def __init__(self, dev):
        self.host = torch.empty(self.INTS, dtype=torch.int32, pin_memory=True)
        self.np = self.host.numpy()
        self.dev = torch.empty(self.INTS, dtype=torch.int32, device=dev)
        self.host_ptr = self.host.data_ptr()
        self.dev_ptr = self.dev.data_ptr()
        addr = ctypes.c_void_p()
        with _device_ctx(dev):
            rc = _hiplib.load().gnf4_hip_host_device_address(self.host_ptr, ctypes.byref(addr))
        # None: the host ring is not mapped for the device (every call copies)
        self.host_dev_ptr = addr.value if rc == 0 else None
        self.events = [None] * self.PARTS
        self.part = 0
        self.off = 0
        self.lock = threading.Lock()

    def stage(self, tables, stream, host_ok=False):
        """Device pointers of `tables` (int sequences / int32 numpy arrays),
        in order (0 for an empty one); None when they do not fit a part.
        `host_ok`: the pointers may address the pinned host ring."""
        lens = [len(t) for t in tables]
        n = sum(lens)
        size = self.INTS // self.PARTS
        if n > size:
            return None
        with self.lock:
            if self.off + n > size:
                ev = self.events[self.part]
                if ev is None:
                    ev = self.events[self.part] = torch.cuda.Event()
                ev.record(stream.torch() if isinstance(stream, _CurStream) else stream)
                self.part = (self.part + 1) % self.PARTS
                self.off = 0
                nxt = self.events[self.part]
                if nxt is not None:
                    nxt.synchronize()
            base = self.part * size + self.off
            direct = host_ok and self.host_dev_ptr is not None
            at = self.host_dev_ptr if direct else self.dev_ptr
            ptrs, b = [], base
            for t, ln in zip(tables, lens):
                if ln:
                    self.np[b:b + ln] = t.numpy() if torch.is_tensor(t) else t
                ptrs.append(at + 4 * b if ln else 0)
                b += ln
            if not direct:
                _hiplib.check(_hiplib.load().gnf4_hip_copy_to_device(
                    self.dev_ptr + 4 * base, self.host_ptr + 4 * base, 4 * n,
                    stream.cuda_stream), "group-table upload")
            self.off += n
            return ptrs


_ARENAS: dict = {}
_RINGS: dict = {}
_TABLE_RINGS: dict = {}
# Creation of the per-device arenas and per-(device, stream) rings: two
# threads making their first call on one stream must get the same ring (a
# dropped ring's pinned block could be reused while a kernel still reads
# group tables from it). Rings are never freed.
_REGISTRY_LOCK = threading.Lock()


def _registered(table, key, make):
    obj = table.get(key)
    if obj is None:
        with _REGISTRY_LOCK:
            obj = table.get(key)
            if obj is None:
                obj = table[key] = make()
    return obj


def _table_ring(dev, stream) -> _TableRing:
    return _registered(_TABLE_RINGS, (str(dev), stream.cuda_stream), lambda: _TableRing(dev))


def _upload_tables(tables, dev, stream, host_ok=False):
    """Device pointers of one launch's int32 tables, and what must stay
    alive until the launch is enqueued: the table ring outside capture
    (`host_ok`: read from its pinned host side), ``to_device_i32``'s
    capture-safe path inside one (or for tables too large for a ring
    part)."""
    if not _PinnedIndexArena._capturing():
        # the capture path's pinned arena must exist before any capture
        # starts (allocating it inside one would invalidate the capture)
        _arena(dev)
        ptrs = _table_ring(dev, stream).stage(tables, stream, host_ok)
        if ptrs is not None:
            return ptrs, None
    views = to_device_i32(tables, dev)
    return [v.data_ptr() if v.numel() else 0 for v in views], views


def _device_ctx(dev):
    """``torch.cuda.device(dev)``, or nothing when dev is already current."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def _arena(device) -> _PinnedIndexArena:
    return _registered(_ARENAS, str(device), lambda: _PinnedIndexArena(device))


def _ring(device, stream) -> _PinnedRing:
    return _registered(_RINGS, (str(device), stream.cuda_stream), _PinnedRing)


def to_device_i32(seqs, device):
    """Small host integer sequences (lists or CPU tensors) to int32 device
    views, in one transfer; one view per input, in order, identical values on
    every path (reference kernel/nf4_grouped.py:229-331). Under graph capture
    the transfer stages through the permanent pinned arena; otherwise through
    an event-guarded pinned ring (asynchronous, no host sync)."""
    lens = [len(s) for s in seqs]
    total = sum(lens)
    dev = torch.device(device)
    if total == 0:
        return [torch.empty(0, dtype=torch.int32, device=dev) for _ in seqs]
    if all(isinstance(s, np.ndarray) for s in seqs):   # the launch paths' tile tables
        flat = np.concatenate([s.astype(np.int32, copy=False) for s in seqs])
    else:
        flat = [int(v) for s in seqs for v in (s.tolist() if torch.is_tensor(s) else s)]
    cuda = dev.type == "cuda" and torch.cuda.is_available()
    if not cuda:
        packed = (torch.from_numpy(flat).to(dev) if isinstance(flat, np.ndarray)
                  else torch.tensor(flat, dtype=torch.int32, device=dev))
    else:
        ar = _arena(dev)   # exists before any capture starts
        capturing = ar._capturing()
        if capturing:
            host, _ = ar.take(total)
            host.copy_(torch.from_numpy(flat) if isinstance(flat, np.ndarray)
                       else torch.tensor(flat, dtype=torch.int32))
            packed = host.to(dev, non_blocking=True)
        else:
            stream = torch.cuda.current_stream(dev)
            packed = _ring(dev, stream).stage(flat, dev, stream)
    out, off = [], 0
    for n in lens:
        out.append(packed[off:off + n])
        off += n
    return out


def _tiles_host(sizes, block_m: int):
    """(t_row0, t_rows, t_group) lists: each group cut into block_m-row tiles;
    empty groups emit nothing. ``sizes`` is only read (``int(m)`` keeps a
    tensor argument from being decremented in place, reference
    kernel/nf4_grouped.py:334-346)."""
    t_row0, t_rows, t_group = [], [], []
    row = 0
    for g, m in enumerate(sizes):
        m = int(m)
        r = 0
        while r < m:
            take = min(block_m, m - r)
            t_row0.append(row + r)
            t_rows.append(take)
            t_group.append(g)
            r += take
        row += m
    return t_row0, t_rows, t_group


def _np_ids(ids):
    """Host expert ids (list, tuple or CPU tensor) as an int32 numpy array."""
    if torch.is_tensor(ids):
        return ids.to(torch.int32).numpy()
    return np.asarray([int(e) for e in ids], dtype=np.int32)


def _largest_first(expert_ids, sizes_i):
    """A decode launch's groups in dispatch order, largest first (stable):
    int32 numpy expert ids [G] and (first row, end row) pairs [2 G] for
    ``gnf4_hip_grouped_decode_pairs``. Each output row is computed on its
    own, so the order changes no bits; it starts the workgroups of the
    groups with the most rows first."""
    sz = np.asarray(sizes_i, dtype=np.int32)
    first = np.zeros(len(sz), dtype=np.int32)
    np.cumsum(sz[:-1], out=first[1:])
    order = np.argsort(-sz, kind="stable")
    pairs = np.empty((len(sz), 2), dtype=np.int32)
    pairs[:, 0] = first[order]
    pairs[:, 1] = first[order] + sz[order]
    return _np_ids(expert_ids)[order], pairs.reshape(-1)


def _tiles_np(sizes_i, block_m: int):
    """``_tiles_host`` as int32 numpy arrays (same tiles, same order), for
    the launch paths: the host planning of a call stays a few numpy ops."""
    m = np.asarray(sizes_i, dtype=np.int64)
    cnt = (m + block_m - 1) // block_m
    n = int(cnt.sum())
    if n == 0:
        z = np.zeros(0, dtype=np.int32)
        return z, z, z
    g = np.repeat(np.arange(len(m), dtype=np.int64), cnt)
    first = np.cumsum(cnt) - cnt                          # first tile of each group
    k = np.arange(n, dtype=np.int64) - first[g]           # tile index within its group
    row0 = (np.cumsum(m) - m)[g] + k * block_m
    rows = np.minimum(block_m, m[g] - k * block_m)
    return row0.astype(np.int32), rows.astype(np.int32), g.astype(np.int32)


def _xcd_balanced(t_row0, t_rows, t_group):
    """Order 256-row tiles for the four-wave kernels, which hand XCD x the
    x-th contiguous eighth of the tile list: the tiles, largest height class
    first (group order within a class), are dealt round robin to 8 bins,
    which then run back to back. Each bin gets an equal share of every
    class and runs its largest tiles first. Only the order changes; every
    output row is computed the same way. O(n), no sort: the input is in group
    order already."""
    n = len(t_row0)
    if n < 16:
        return t_row0, t_rows, t_group
    if isinstance(t_rows, np.ndarray):
        cls = (t_rows > 128).astype(np.int8) * 2 + ((t_rows > 64) & (t_rows <= 128))
        ranked = np.concatenate([np.nonzero(cls == c)[0] for c in (2, 1, 0)])
        order = np.concatenate([ranked[x::8] for x in range(8)])
        return t_row0[order], t_rows[order], t_group[order]
    by_class = ([], [], [])
    for i, r in enumerate(t_rows):
        by_class[2 if r > 128 else (1 if r > 64 else 0)].append(i)
    ranked = by_class[2] + by_class[1] + by_class[0]
    order = [i for x in range(8) for i in ranked[x::8]]
    return ([t_row0[i] for i in order], [t_rows[i] for i in order],
            [t_group[i] for i in order])


def build_group_tiles(sizes, block_m: int, device):
    """Expand jagged group sizes into fixed M-tiles: ``(row0, valid_rows,
    group_idx)`` int32 device tensors, one transfer for all three
    (reference kernel/nf4_grouped.py:334-362)."""
    a, b, c = to_device_i32(_tiles_host(sizes, block_m), device)
    return a, b, c


# --------------------------------------------------------------------- plan --

_LUT_CACHE: dict = {}
_SM_CACHE: dict = {}


def _sm_count(device) -> int:
    """Compute-unit count of ``device`` (the reference's SM count query,
    kernel/nf4_grouped.py:581-591); 64 when no GPU is visible."""
    key = str(device)
    if key not in _SM_CACHE:
        if torch.cuda.is_available() and "cuda" in key:
            _SM_CACHE[key] = torch.cuda.get_device_properties(device).multi_processor_count
        else:
            _SM_CACHE[key] = 64
    return _SM_CACHE[key]


def _decode_plan(N: int, K: int, T: int, sm_count: int):
    """Decode plan ``(BLOCK_N, num_warps, split_k)`` with the reference's rule
    (kernel/nf4_grouped.py:609-632): the constant (64, 2) and split-K only for
    starved grids (programs < 2 * SMs), power of two up to 8, each split owning
    at least SPLITK_MIN_BLOCKS absmax blocks. The HIP decode kernel streams
    whole rows per wave and does not use the numbers; the function is kept for
    callers and for ``decode_dispatch``."""
    bn, warps = 64, 2
    programs = T * -(-N // bn)
    split_k = 1
    if programs < 2 * sm_count:
        want = -(-(4 * sm_count) // programs)
        while split_k < want and split_k < 8:
            split_k *= 2
        kblocks = max(K // BLOCKSIZE, 1)
        while split_k > 1 and kblocks // split_k < SPLITK_MIN_BLOCKS:
            split_k //= 2
    return bn, warps, split_k


def decode_dispatch(N: int, K: int, T: int, sm_count: int):
    """``("dequant",)`` below the fused floor, else ``("fused", BLOCK_N,
    num_warps, split_k)`` (reference kernel/nf4_grouped.py:635-649). The op
    itself always runs fused; integrations consult this helper."""
    traffic = T * N * (K // 2 + K // 16)
    if traffic < DECODE_MIN_FUSED_BYTES:
        return ("dequant",)
    return ("fused", *_decode_plan(N, K, T, sm_count))


def _lut(device):
    key = str(device)
    if key not in _LUT_CACHE:
        _LUT_CACHE[key] = torch.tensor(NF4_LUT, dtype=torch.float32, device=device)
    return _LUT_CACHE[key]


def _prefill_block_m(max_rows: int) -> int:
    """Group-size-keyed M-tile height (reference kernel/nf4_grouped.py:686-694)."""
    if max_rows <= 16:
        return 16
    if max_rows <= 32:
        return 32
    if max_rows <= 64:
        return 64
    return 128


_SUPPORTED_BLOCK_M = (16, 32, 64, 128, 256)


def _kernel_block_m(block_m: int) -> int:
    """The smallest supported tile height >= block_m (tiling never changes
    what an output row is, only how rows are batched)."""
    for bm in _SUPPORTED_BLOCK_M:
        if block_m <= bm:
            return bm
    return 128


def _auto_block_m(max_rows: int, K: int = 0) -> int:
    """Tile height the forward uses when the caller names none: the
    reference's group-size rule (``_prefill_block_m``), except that groups of
    more than 128 rows, and any tiled call with K >= 1024, take the 256-row
    tiles of the four-wave kernel (each decoded weight feeds up to twice the
    rows; its tile prologue is paid back over a long K; the bits are the
    same). Measured, 128 experts, Qwen3 shapes: K = 2048 runs 5-11 % faster
    on 256-row tiles at 24-128 rows per group, K = 768 0-4 % slower at
    100-128 rows."""
    if max_rows > 128 or K >= 1024:
        return 256
    return _kernel_block_m(_prefill_block_m(max_rows))


def _tall_tiles_ok(N: int, K: int) -> bool:
    """Whether the library takes 256-row forward tiles for this shape (whole
    64-wide k steps, 4-column output stores)."""
    return K % 64 == 0 and N % 4 == 0


def _fwd_block_m(max_m: int, N: int, K: int, block_m=None) -> int:
    """Tile height of a tiled forward launch, shared by the op and by
    ``GroupPlan``: the caller's ``block_m`` rounded up to a supported
    height, else ``_auto_block_m`` where the shape takes 256-row tiles, else
    the reference's group-size rule."""
    if block_m is not None:
        return _kernel_block_m(block_m)
    bm = _auto_block_m(max_m, K)
    if bm == 256 and not _tall_tiles_ok(N, K):
        bm = _kernel_block_m(_prefill_block_m(max_m))
    return bm


# ------------------------------------------------------------------ launch --

def _require_gpu(t: torch.Tensor, op: str, hint: str):
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{op} runs the HIP kernel and requires CUDA tensors (ROCm devices "
            f"report type 'cuda'; got device '{t.device.type}'). {hint}")


def _aligned_rows(t: torch.Tensor, align: int) -> torch.Tensor:
    """Packed weights with a contiguous last dimension and row/expert strides
    (and base) aligned to ``align`` bytes; a misaligned view is copied."""
    if (t.stride(-1) != 1 or t.stride(1) % align or t.stride(0) % align
            or t.data_ptr() % align):
        return t.contiguous()
    return t


def _scales_view(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _act_view(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
        return t.contiguous()
    return t


_WIDEN_DTYPES = {torch.float16: _hiplib.DTYPE_F16, torch.float32: _hiplib.DTYPE_F32}


def _bf16_activations(a_cat: torch.Tensor, op: str) -> torch.Tensor:
    """bf16 activations for the forward kernels. fp16 and fp32 inputs (the
    reference accepts both, kernel/nf4_grouped.py:456-458) are rounded to bf16
    once, nearest-even, by the library's widening kernel; any other dtype is
    a TypeError."""
    if a_cat.dtype == torch.bfloat16:
        return _act_view(a_cat)
    code = _WIDEN_DTYPES.get(a_cat.dtype)
    if code is None:
        raise TypeError(f"{op}: activations must be bfloat16, float16 or float32, "
                        f"got {a_cat.dtype}")
    src = _act_view(a_cat)
    T, K = src.shape
    dst = torch.empty(T, K, dtype=torch.bfloat16, device=src.device)
    with torch.cuda.device(src.device):
        rc = _hiplib.load().gnf4_hip_activations_to_bf16(
            src.data_ptr(), code, T, K, src.stride(0), dst.data_ptr(), dst.stride(0),
            _stream_ptr(src.device))
    _hiplib.check(rc, op)
    return dst


def _eids_device(expert_ids, dev):
    """Expert ids as int32 on ``dev``: a device tensor passes through; a list
    or host tensor converts once (same values on every path)."""
    if torch.is_tensor(expert_ids) and expert_ids.is_cuda:
        return expert_ids.to(device=dev, dtype=torch.int32)
    return None


def _check_host_ids(expert_ids, E: int) -> None:
    """Host-side expert ids must index the stack: an out-of-range id would
    make the kernel read outside the weights. Device-resident ids are the
    caller's responsibility (checking them would synchronise)."""
    ids = expert_ids.tolist() if torch.is_tensor(expert_ids) else expert_ids
    if len(ids) and (int(min(ids)) < 0 or int(max(ids)) >= E):
        raise ValueError(f"expert id out of range [0, {E})")


class _CurStream:
    """The current stream of a device as a raw handle, read through torch's
    C binding (``torch.cuda.current_stream`` builds a Python stream object per
    call, several microseconds of a decode call's host time). ``torch()``
    gives the stream object where one is needed (event records)."""

    __slots__ = ("dev", "cuda_stream")

    def __init__(self, dev):
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        self.dev = dev
        self.cuda_stream = torch._C._cuda_getCurrentRawStream(idx)

    def torch(self):
        return torch.cuda.current_stream(self.dev)


def _stream_ptr(dev) -> int:
    return _CurStream(dev).cuda_stream


class GroupPlan:
    """Device-resident group tables for repeated calls with the same routing
    (e.g. inside a captured graph or a timing loop): the expert ids, row
    offsets or tile table are uploaded once, so a planned call launches the
    kernel with no host-to-device copy. Not part of the reference's API.

    The tiled path's tile height depends on the weights' shape (as in the
    op, ``_fwd_block_m``); its tables are built on the first planned launch
    for a shape, or up front for ``shape=(N, K)``. A graph capture must be
    preceded by one eager planned launch per shape (uploads synchronise)."""

    def __init__(self, sizes, expert_ids, device, block_m=None, shape=None):
        sizes_i = [int(m) for m in sizes]
        self.sizes = sizes_i
        self.G = len(sizes_i)
        self.max_m = max(sizes_i) if sizes_i else 0
        self.one_row_each = bool(sizes_i) and min(sizes_i) == 1 and self.max_m == 1
        self.device = torch.device(device)
        ids = expert_ids.tolist() if torch.is_tensor(expert_ids) else list(expert_ids)
        self.max_id = max((int(e) for e in ids), default=-1)
        self.min_id = min((int(e) for e in ids), default=0)
        self.user_block_m = block_m
        self.decode = self.max_m <= DECODE_MAX_ROWS and block_m is None
        self.eids = torch.tensor(ids, dtype=torch.int32, device=self.device)
        self.host_ids = np.asarray([int(e) for e in ids], dtype=np.int32)
        self.host_row_off = None
        self.eids_lf = self.row_pairs = None
        self._tables = {}
        if self.decode:
            row_off = [0]
            for m in sizes_i:
                row_off.append(row_off[-1] + m)
            self.row_off = torch.tensor(row_off, dtype=torch.int32, device=self.device)
            if not self.one_row_each:
                self.host_row_off = np.asarray(row_off, dtype=np.int32)
                # the launches that leave the GEMV classes take the groups
                # largest first (gnf4_hip_grouped_decode_pairs)
                ids_lf, pairs = _largest_first(self.host_ids, sizes_i)
                self.eids_lf = torch.from_numpy(ids_lf).to(self.device)
                self.row_pairs = torch.from_numpy(pairs).to(self.device)
        else:
            self.row_off = None
            if shape is not None:
                self.tables(*shape)

    def tables(self, N: int, K: int):
        """(block_m, (t_row0, t_rows, t_group) on the device) for a weight
        shape: the tile height the op would use."""
        bm = _fwd_block_m(self.max_m, N, K, self.user_block_m)
        if bm not in self._tables:
            t0, tr, tg = _tiles_host(self.sizes, bm)
            if bm == 256:
                t0, tr, tg = _xcd_balanced(t0, tr, tg)
            self._tables[bm] = tuple(torch.tensor(v, dtype=torch.int32, device=self.device)
                                     for v in (t0, tr, tg))
        return bm, self._tables[bm]

    def args(self, N: int, K: int):
        if self.decode:
            ro = None if self.one_row_each else self.row_off.data_ptr()
            return (self.eids.data_ptr(), ro, self.G, None, None, None, 0, self.max_m)
        bm, (t0, tr, tg) = self.tables(N, K)
        return (self.eids.data_ptr(), None, self.G, t0.data_ptr(), tr.data_ptr(), tg.data_ptr(),
                t0.numel(), bm)


def launch_planned(fmt: int, a_cat, W, S, plan: GroupPlan, out=None):
    """Forward launch with a prepared GroupPlan: the kernel and nothing else."""
    lib = _hiplib.load()
    E, N, half = W.shape
    T, K = a_cat.shape
    dev = a_cat.device
    if plan.min_id < 0 or plan.max_id >= E:
        raise ValueError(f"expert id out of range [0, {E})")
    a_cat, W, S = (_bf16_activations(a_cat, "launch_planned"), _aligned_rows(W, 16),
                   _scales_view(S))
    if out is None:
        out = torch.empty(T, N, dtype=torch.bfloat16, device=dev)
    if plan.decode and 0 < plan.G <= IDS_ARG_MAX:
        ro = plan.host_row_off
        with torch.cuda.device(dev):
            rc = lib.gnf4_hip_grouped_decode_ids(
                fmt, a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
                W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
                plan.host_ids.ctypes.data, ro.ctypes.data if ro is not None else None, plan.G,
                plan.max_m, N, K, out.data_ptr(), out.stride(0), _stream_ptr(dev))
        if rc != 1:
            _hiplib.check(rc, "launch_planned")
            return out
    if plan.decode and plan.G > 0 and plan.row_pairs is not None:
        with torch.cuda.device(dev):
            rc = lib.gnf4_hip_grouped_decode_pairs(
                fmt, a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
                W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
                plan.eids_lf.data_ptr(), plan.row_pairs.data_ptr(), plan.G, plan.max_m,
                N, K, out.data_ptr(), out.stride(0), _stream_ptr(dev))
        _hiplib.check(rc, "launch_planned")
        return out
    with torch.cuda.device(dev):
        rc = lib.gnf4_hip_grouped_fwd(
            fmt, a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
            W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
            *plan.args(N, K), N, K, out.data_ptr(), out.stride(0), _stream_ptr(dev))
    _hiplib.check(rc, "launch_planned")
    return out


def _launch_fwd(fmt: int, a_cat, W, S, sizes, expert_ids, block_m, op, fp32w=False):
    """Shared forward launcher for NF4 and MXFP4. ``fp32w`` (NF4): tiled
    launches take the fp32-weight tiles (``gnf4_hip_nf4_fwd_fp32w``, the
    reference's VARIANT 1), at most 64 rows per tile."""
    lib = _hiplib.load()
    E, N, half = W.shape
    T, K = a_cat.shape
    dev = a_cat.device
    out = torch.empty(T, N, dtype=torch.bfloat16, device=dev)
    G = len(sizes)
    if T == 0 or G == 0:
        return out
    a_cat = _bf16_activations(a_cat, op)
    W = _aligned_rows(W, 16)
    S = _scales_view(S)
    sizes_i = [int(m) for m in sizes]
    max_m = max(sizes_i)
    eids_dev = _eids_device(expert_ids, dev)
    if eids_dev is None:
        _check_host_ids(expert_ids, E)
    host_eids = [] if eids_dev is not None else expert_ids
    stream = _CurStream(dev)
    if max_m <= DECODE_MAX_ROWS and block_m is None and eids_dev is None and G <= IDS_ARG_MAX:
        # host ids: in the kernel's arguments where a GEMV class takes the
        # launch (no table read ahead of the weights, no upload)
        ids32 = _np_ids(expert_ids)
        ro = None
        if not (min(sizes_i) == 1 and max_m == 1):
            ro = np.zeros(G + 1, dtype=np.int32)
            np.cumsum(np.asarray(sizes_i, dtype=np.int32), out=ro[1:])
        with _device_ctx(dev):
            rc = lib.gnf4_hip_grouped_decode_ids(
                fmt, a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
                W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
                ids32.ctypes.data, ro.ctypes.data if ro is not None else None, G, max_m,
                N, K, out.data_ptr(), out.stride(0), stream.cuda_stream)
        if rc != 1:
            _hiplib.check(rc, op)
            return out
    if max_m <= DECODE_MAX_ROWS and block_m is None:
        if min(sizes_i) == 1 and max_m == 1:
            # one row per group: group g is row g, no offset table to upload
            (e_p,), keep = _upload_tables((host_eids,), dev, stream, host_ok=True)
            r_ptr = None
        elif eids_dev is None:
            # host ids: the groups largest first, as (first, end) row pairs
            ids_lf, pairs = _largest_first(expert_ids, sizes_i)
            (e_p, p_p), keep = _upload_tables((ids_lf, pairs), dev, stream, host_ok=True)
            with _device_ctx(dev):
                rc = lib.gnf4_hip_grouped_decode_pairs(
                    fmt, a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
                    W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0),
                    S.stride(1), e_p, p_p, G, max_m, N, K, out.data_ptr(), out.stride(0),
                    stream.cuda_stream)
            del keep
            _hiplib.check(rc, op)
            return out
        else:
            row_off = [0]
            for m in sizes_i:
                row_off.append(row_off[-1] + m)
            (e_p, r_ptr), keep = _upload_tables((host_eids, row_off), dev, stream,
                                                host_ok=True)
        e_ptr = eids_dev.data_ptr() if eids_dev is not None else e_p
        # decode path: block_m carries the largest group size
        args = (e_ptr, r_ptr, G, None, None, None, 0, max_m)
    elif fp32w:
        bm = min(_kernel_block_m(block_m if block_m is not None else _prefill_block_m(max_m)), 64)
        t0, tr, tg = _tiles_np(sizes_i, bm)
        (e_p, t0_p, tr_p, tg_p), keep = _upload_tables((_np_ids(host_eids), t0, tr, tg), dev,
                                                       stream)
        e_ptr = eids_dev.data_ptr() if eids_dev is not None else e_p
        with _device_ctx(dev):
            rc = lib.gnf4_hip_nf4_fwd_fp32w(
                a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
                W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
                e_ptr, t0_p, tr_p, tg_p, len(t0), bm, N, K, out.data_ptr(), out.stride(0),
                stream.cuda_stream)
        del keep, eids_dev
        _hiplib.check(rc, op)
        return out
    else:
        bm = _fwd_block_m(max_m, N, K, block_m)
        t0, tr, tg = _tiles_np(sizes_i, bm)
        if bm == 256:
            t0, tr, tg = _xcd_balanced(t0, tr, tg)
            if len(t0) <= ARG_TILES_MAX:
                a0, ar, ag, is_e, e_ptr = _arg_tiles(t0, tr, tg, eids_dev, expert_ids)
                with _device_ctx(dev):
                    rc = lib.gnf4_hip_grouped_fwd_tiles(
                        fmt, a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
                        W.data_ptr(), W.stride(0), W.stride(1),
                        S.data_ptr(), S.stride(0), S.stride(1),
                        e_ptr, a0.ctypes.data, ar.ctypes.data, ag.ctypes.data, is_e, len(a0),
                        N, K, out.data_ptr(), out.stride(0), stream.cuda_stream)
                if rc != 1:
                    del eids_dev
                    _hiplib.check(rc, op)
                    return out
        (e_p, t0_p, tr_p, tg_p), keep = _upload_tables((_np_ids(host_eids), t0, tr, tg), dev,
                                                       stream)
        e_ptr = eids_dev.data_ptr() if eids_dev is not None else e_p
        args = (e_ptr, None, G, t0_p, tr_p, tg_p, len(t0), bm)
    with _device_ctx(dev):
        rc = lib.gnf4_hip_grouped_fwd(
            fmt, a_cat.data_ptr(), _hiplib.DTYPE_BF16, a_cat.stride(0),
            W.data_ptr(), W.stride(0), W.stride(1),
            S.data_ptr(), S.stride(0), S.stride(1),
            *args, N, K, out.data_ptr(), out.stride(0), stream.cuda_stream)
    del keep, eids_dev  # index tensors stay alive until the launch is enqueued
    _hiplib.check(rc, op)
    return out


def _dgrad_block_m(max_rows: int, N: int, K: int) -> int:
    """Tile height of a dgrad launch: 256-row tiles when the four-wave
    transposed-read kernel takes the shape (whole 64-wide n steps and k
    blocks), else the forward's group-size rule capped at 128 rows (the
    eight-wave dgrad kernels)."""
    if max_rows > 128 and N % 64 == 0 and K % 64 == 0:
        return 256
    return _kernel_block_m(_prefill_block_m(max_rows))


# Decode launches of at most this many groups with host-known expert ids pass
# the ids (and row offsets) in the GEMV kernels' arguments
# (gnf4_hip_grouped_decode_ids).
IDS_ARG_MAX = 384

# Tile tables of at most this many m-tiles travel in the kernel arguments of
# the 256-row kernels (gnf4_hip_grouped_fwd_tiles / _dgrad_tiles): no upload,
# so no copy is enqueued ahead of the launch (in a captured graph: no copy
# node and no dependency gap before the kernel).
ARG_TILES_MAX = 256


def _arg_tiles(t0, tr, tg, eids_dev, expert_ids):
    """(row0, rows, group-or-expert, group_is_expert, expert-ids pointer) as
    contiguous int32 host arrays for the kernel-argument table: with host
    ids each tile carries its expert id, with device ids its group index."""
    c = lambda x: np.ascontiguousarray(x, dtype=np.int32)
    if eids_dev is not None:
        return c(t0), c(tr), c(tg), 0, eids_dev.data_ptr()
    return c(t0), c(tr), c(_np_ids(expert_ids)[tg]), 1, None


def _launch_dgrad(fmt: int, grad_out, W, S, sizes, expert_ids, op):
    lib = _hiplib.load()
    E, N, half = W.shape
    K = half * 2
    T = grad_out.shape[0]
    dev = grad_out.device
    out = torch.empty(T, K, dtype=torch.bfloat16, device=dev)
    G = len(sizes)
    if T == 0 or G == 0:
        return out
    g = _act_view(grad_out)
    W = _aligned_rows(W, 4)
    S = _scales_view(S)
    sizes_i = [int(m) for m in sizes]
    # tile height from the largest group, as in the forward (the kernel's
    # per-row arithmetic does not depend on it)
    bm = _dgrad_block_m(max(sizes_i), N, K)
    t0, tr, tg = _tiles_np(sizes_i, bm)
    if bm == 256:
        t0, tr, tg = _xcd_balanced(t0, tr, tg)
    eids_dev = _eids_device(expert_ids, dev)
    if eids_dev is None:
        _check_host_ids(expert_ids, E)
    stream = _CurStream(dev)
    if bm == 256 and len(t0) <= ARG_TILES_MAX:
        a0, ar, ag, is_e, e_ptr = _arg_tiles(t0, tr, tg, eids_dev, expert_ids)
        with _device_ctx(dev):
            rc = lib.gnf4_hip_grouped_dgrad_tiles(
                fmt, g.data_ptr(), _hiplib.DTYPE_BF16, g.stride(0),
                W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
                e_ptr, a0.ctypes.data, ar.ctypes.data, ag.ctypes.data, is_e, len(a0),
                N, K, out.data_ptr(), out.stride(0), stream.cuda_stream)
        if rc != 1:
            del eids_dev
            _hiplib.check(rc, op)
            return out
    (e_p, t0_p, tr_p, tg_p), keep = _upload_tables(
        (_np_ids([] if eids_dev is not None else expert_ids), t0, tr, tg), dev, stream)
    e_ptr = eids_dev.data_ptr() if eids_dev is not None else e_p
    with _device_ctx(dev):
        rc = lib.gnf4_hip_grouped_dgrad(
            fmt, g.data_ptr(), _hiplib.DTYPE_BF16, g.stride(0),
            W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
            e_ptr, t0_p, tr_p, tg_p, len(t0), bm,
            N, K, out.data_ptr(), out.stride(0), stream.cuda_stream)
    del keep, eids_dev
    _hiplib.check(rc, op)
    return out


# ------------------------------------------------------------------ forward --

_PREFILL_VARIANTS = (0, 1, 3)


def gemm_4bit_grouped(
    a_cat,
    B,
    absmax,
    sizes,
    expert_ids,
    block_m: int | None = None,
    decode_config: tuple | None = None,
    split_k: int | None = None,
    prefill_config: tuple | None = None,
    prefill_variant: int | None = None,
    prefill_groups: int = 1,
):
    """Single-launch grouped NF4 GEMM (reference kernel/nf4_grouped.py:697-907).

    ``a_cat [T, K]`` bf16 (fp16 and fp32 are rounded to bf16 first),
    group-sorted; ``B [E, N, K//2]`` uint8;
    ``absmax [E, N, K//64]`` fp32; ``sizes`` per-group row counts (a list or
    tensor, read only; zero-size groups are allowed); ``expert_ids [G]`` as a
    list, CPU tensor or device tensor (all give identical bits). Returns
    ``[T, N]`` bf16 in the same group order.

    Path: groups of at most 16 rows (always when ``max(sizes) == 1``) take the
    decode kernel, which streams each active expert's weights once; larger
    groups take the tiled MFMA kernel with ``block_m`` (default
    ``_prefill_block_m(max(sizes))``). An explicit ``block_m`` forces the tiled
    kernel for groups above one row.

    The reference's tuning knobs are accepted and validated so call sites keep
    working: ``decode_config`` (BLOCK_N, num_warps), ``split_k`` (>= 1),
    ``prefill_config`` (BLOCK_N, num_warps, num_stages) and
    ``prefill_groups`` (1 or 2). They select Triton schedules in the
    reference; here one HIP mainloop serves them all and they change neither
    the path nor the result.

    ``prefill_variant`` (0, 1 or 3) picks the tiled path's weight precision
    as in the reference (kernel/nf4_grouped.py:438-452): ``None``, 0 and 3
    run the default tiles, which round each decoded weight LUT x absmax to
    bf16 once (the reference's VARIANT 3); 1 runs the fp32-weight tiles
    (bf16 hi + lo parts of the fp32 weight, two MFMAs per slice: VARIANT 1's
    fp32 weights) at about twice the matrix work. Decode-path calls (groups
    of at most 16 rows, no ``block_m``) are fp32-accurate either way.
    """
    E, N, _ = B.shape
    T, K = a_cat.shape
    assert sum(int(m) for m in sizes) == T, (sum(int(m) for m in sizes), T)
    dev = a_cat.device
    _require_gpu(
        a_cat, "gemm_4bit_grouped",
        "For a CPU-checkable decode of the same NF4 bytes, use "
        "dequant_ref(packed, absmax, N, K) -- the pure-torch reference decode.")
    if B.dtype != torch.uint8:
        raise TypeError(f"B must be uint8 packed nibbles, got {B.dtype}")
    if absmax.dtype != torch.float32:
        raise TypeError(f"absmax must be float32, got {absmax.dtype}")
    if K % BLOCKSIZE or B.shape[2] * 2 != K:
        raise ValueError(f"K={K} must equal 2*B.shape[2]={2 * B.shape[2]} and be a "
                         f"multiple of {BLOCKSIZE}")
    if tuple(absmax.shape) != (E, N, K // BLOCKSIZE):
        raise ValueError(f"absmax shape {tuple(absmax.shape)} != {(E, N, K // BLOCKSIZE)}")
    if len(sizes) != len(expert_ids):
        raise ValueError(f"{len(sizes)} group sizes but {len(expert_ids)} expert ids")
    if decode_config is not None and len(tuple(decode_config)) != 2:
        raise ValueError(f"decode_config must be (BLOCK_N, num_warps), got {decode_config}")
    if split_k is not None and int(split_k) < 1:
        raise ValueError(f"split_k must be >= 1, got {split_k}")
    if prefill_config is not None and len(tuple(prefill_config)) != 3:
        raise ValueError("prefill_config must be (BLOCK_N, num_warps, num_stages), "
                         f"got {prefill_config}")
    if prefill_variant is not None and prefill_variant not in _PREFILL_VARIANTS:
        raise ValueError(f"prefill_variant {prefill_variant} is not one of {_PREFILL_VARIANTS}")
    if prefill_groups not in (1, 2):
        raise ValueError(f"prefill_groups must be 1 or 2, got {prefill_groups}")
    if prefill_groups == 2 and K % (2 * BLOCKSIZE):
        raise ValueError(f"prefill_groups=2 needs K % {2 * BLOCKSIZE} == 0, got K={K}")
    if B.device != dev or absmax.device != dev:
        raise ValueError("a_cat, B and absmax must be on the same device")
    bm = block_m if (block_m is not None and max((int(m) for m in sizes), default=0) > 1) else None
    return _launch_fwd(_hiplib.FMT_NF4, a_cat, B, absmax, sizes, expert_ids, bm,
                       "gemm_4bit_grouped", fp32w=prefill_variant == 1)


def dequant_ref(packed_row_major: torch.Tensor, absmax: torch.Tensor, N: int, K: int):
    """Plain-torch decode ``w[n, k] = NF4[code(n, k)] * absmax[n, k // 64]``
    in fp32 (one rounding), element 2j from the high nibble of byte j
    (reference kernel/nf4_grouped.py:910-929). Runs on any device; it is the
    checkable decode the CPU refusal points callers to."""
    b = packed_row_major.reshape(N, K // 2).to(torch.int64)
    idx = torch.stack((b >> 4, b & 0xF), dim=-1).reshape(N, K // BLOCKSIZE, BLOCKSIZE)
    scale = absmax.reshape(N, K // BLOCKSIZE, 1).to(torch.float32)
    return (_lut(packed_row_major.device)[idx] * scale).reshape(N, K)


# -------------------------------------------------------------------- dgrad --

def dgrad_eligible(grad_out, B, absmax, block_k: int = 64):
    """None if this problem can take the dgrad kernel, else the reason
    (reference kernel/nf4_grouped.py:1034-1053)."""
    if grad_out.dtype != torch.bfloat16:
        return f"grad_out dtype {grad_out.dtype} is not bfloat16"
    if BLOCKSIZE % block_k:
        return f"BLOCK_K {block_k} does not divide the quant blocksize {BLOCKSIZE}"
    K = B.shape[2] * 2
    if K % block_k:
        return f"K {K} not divisible by BLOCK_K {block_k}"
    if absmax.shape[2] * BLOCKSIZE != K:
        return f"absmax blocks {absmax.shape[2]} do not tile K {K} at blocksize {BLOCKSIZE}"
    if B.numel() == 0:
        return "packed storage is empty (evicted?)"
    return None


def dgrad_4bit_grouped(grad_out, B, absmax, sizes, expert_ids, config=None):
    """``grad_a[t, :] = grad_out[t, :] @ dequant_nf4(B[e(t)])`` in one launch
    (reference kernel/nf4_grouped.py:1056-1121). ``grad_out [T, N]`` bf16
    group-sorted; returns ``[T, K]`` bf16. The weights are read through the
    same ``[E, N, K/2]`` layout as the forward (no transposed copy).

    ``config`` = (BLOCK_M, BLOCK_N, BLOCK_K, num_warps): BLOCK_K must divide
    64 (eligibility); the other entries steer the reference's Triton schedule
    and are accepted unused. The kernel's tiles and its fixed ascending
    64-wide contraction over N do not depend on the config, so the output is
    bitwise independent of it."""
    E, N, half = B.shape
    K = half * 2
    T = grad_out.shape[0]
    assert sum(int(m) for m in sizes) == T, (sum(int(m) for m in sizes), T)
    _require_gpu(
        grad_out, "dgrad_4bit_grouped",
        "The CPU-checkable equivalent is grad_out @ dequant_ref(packed, absmax, N, K) "
        "per group.")
    _block_m, _block_n, block_k, _warps = config or _DGRAD_DEFAULT
    why = dgrad_eligible(grad_out, B, absmax, block_k)
    if why is not None:
        raise ValueError(
            f"dgrad_4bit_grouped cannot run this problem: {why}. Callers that can "
            "fall back should check dgrad_eligible() first rather than catching this.")
    if grad_out.shape[1] != N:
        raise ValueError(f"grad_out has {grad_out.shape[1]} columns, B has N={N}")
    if absmax.dtype != torch.float32 or tuple(absmax.shape) != (E, N, K // BLOCKSIZE):
        raise ValueError(f"absmax must be float32 {(E, N, K // BLOCKSIZE)}, got "
                         f"{absmax.dtype} {tuple(absmax.shape)}")
    if len(sizes) != len(expert_ids):
        raise ValueError(f"{len(sizes)} group sizes but {len(expert_ids)} expert ids")
    return _launch_dgrad(_hiplib.FMT_NF4, grad_out, B, absmax, sizes, expert_ids,
                         "dgrad_4bit_grouped")
