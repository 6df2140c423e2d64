"""Device-side MoE routing around the grouped NF4 expert GEMM.

The reference routes on the host side of its kernels: the MoE block sorts
(token, slot) rows by expert, counts them, hands ``sizes`` / ``expert_ids``
lists to the grouped op, then unsorts and weights the outputs
(kernel/arena_moe_patch.py:41-66); its router top-k + softmax epilogue is a
CPU C routine (gnf4_route_epilogue_bf16, gnf4_native/cpu_kernels.c:1408-1471).
Here every step is a HIP kernel, so a decode MoE layer
    logits -> top-k -> group -> gather -> expert FFN -> combine
never reads the routing on the host and can be captured in one graph:

  * ``route_topk``   top-k selection (stable descending, ties to the lower
    index) with the reference's two softmax modes, bf16 weights;
  * ``route_groups`` the stable sort by expert: device tables (expert ids,
    row offsets) sized for ``slots = min(T * k, E)`` groups, so the decode
    kernels can be launched without knowing how many experts are active
    (empty groups exit at once);
  * ``gather_rows`` / ``combine`` the row gather into group order and the
    weighted unsort-and-sum;
  * ``moe_ffn`` (given top-k ids and weights) and ``moe_layer`` (given
    router logits) the whole expert layer. At decode (T <= 16 tokens) the
    top-k, grouping and gather run as ONE launch (``gnf4_hip_route_decode``),
    then the fused expert FFN, then the combine: three launches per layer.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

import _hiplib
import nf4_ffn
import nf4_grouped
from nf4_grouped import DECODE_MAX_ROWS, _aligned_rows, _require_gpu, _scales_view, _stream_ptr

ROUTE_MAX_K = 64          # as the reference's epilogue
ROUTE_MAX_EXPERTS = 512   # grouping kernel's LDS tables
# Largest group of the device-routed decode path: an expert's rows beyond it
# form further groups, so the expert FFN launches in the class of at most 8
# rows (the split-table kernels' one row set) instead of T rows (two row
# sets at T > 8; Qwen3 batch 16: 123 us -> about the host-routed 67 us)
DECODE_GROUP_CAP = 8


def route_slots(N: int, E: int, cap: int = 0) -> int:
    """Group-table size that holds every routing of N rows over E experts
    with groups of at most ``cap`` rows (0: one group per expert)."""
    M = min(N, E)
    return max(1, M + ((N - M) // cap if cap > 0 else 0))


def _dev_check(t, op):
    _require_gpu(t, op, "The CPU forms are the reference's cpu_grouped.route_epilogue_bf16 "
                        "and its MoE block's sort; a checkable weight decode is "
                        "dequant_ref(packed, absmax, N, K).")


def route_topk(logits: torch.Tensor, k: int, mode: int = 0, norm: bool = False):
    """Top-k experts and their bf16 weights per token, from router logits
    ``[T, E]`` (fp32; bf16 / fp16 are widened exactly). ``mode`` 0: softmax
    over all E logits gathered at the selection (renormalised over it when
    ``norm``, olmoe / qwen3); 1: softmax over the k selected logits (gpt_oss).
    Returns ``(ids int64 [T, k], weights bf16 [T, k])`` in selection order."""
    _dev_check(logits, "route_topk")
    if logits.dim() != 2:
        raise ValueError(f"logits must be [T, E], got {tuple(logits.shape)}")
    T, E = logits.shape
    if not (1 <= k <= min(E, ROUTE_MAX_K)):
        raise ValueError(f"k={k} must be in [1, min(E={E}, {ROUTE_MAX_K})]")
    if mode not in (0, 1):
        raise ValueError(f"mode must be 0 or 1, got {mode}")
    lg = logits.float()
    if lg.stride(-1) != 1:
        lg = lg.contiguous()
    idx = torch.empty(T, k, dtype=torch.int64, device=lg.device)
    wts = torch.empty(T, k, dtype=torch.bfloat16, device=lg.device)
    with torch.cuda.device(lg.device):
        rc = _hiplib.load().gnf4_hip_route_topk(
            lg.data_ptr(), T, E, lg.stride(0), k, mode, int(bool(norm)), idx.data_ptr(), k,
            wts.data_ptr(), k, _stream_ptr(lg.device))
    _hiplib.check(rc, "route_topk")
    return idx, wts


@dataclass
class RoutePlan:
    """Device tables of one routing: ``eids [slots]``, ``row_off [slots + 1]``
    (groups past the active count are empty), ``order [N]`` (grouped
    position -> routed row t * k + j), ``pos [N]`` (its inverse) and
    ``info [3]`` (active groups, largest group, bad-id flag). ``cap``: the
    largest group the grouping allowed (0: one group per expert)."""
    eids: torch.Tensor
    row_off: torch.Tensor
    order: torch.Tensor
    pos: torch.Tensor
    info: torch.Tensor
    T: int
    k: int
    E: int
    slots: int
    cap: int = 0

    @property
    def rows(self) -> int:
        return self.T * self.k

    def max_rows_bound(self) -> int:
        """An upper bound of the largest group known without a device read:
        an expert appears at most once per token when the top-k ids of a
        token are distinct (as the selection guarantees), and no group
        exceeds the grouping's cap."""
        b = min(self.T, self.rows)
        return min(b, self.cap) if self.cap > 0 else b

    def host_groups(self):
        """(sizes, expert_ids) of the active groups as host lists. Reads the
        device (synchronises); the decode path never calls it."""
        n = int(self.info[0].item())
        off = self.row_off[:n + 1].tolist()
        return [off[g + 1] - off[g] for g in range(n)], self.eids[:n].tolist()

    def bad_ids(self) -> bool:
        """True if an expert id was outside [0, E) (reads the device)."""
        return bool(self.info[2].item())


def route_groups(topk_ids: torch.Tensor, n_experts: int, slots: int | None = None,
                 cap: int = 0) -> RoutePlan:
    """Group the T * k routed rows by expert on the device (one launch);
    ``cap`` > 0 splits an expert's rows into groups of at most cap rows."""
    _dev_check(topk_ids, "route_groups")
    if topk_ids.dim() != 2:
        raise ValueError(f"topk_ids must be [T, k], got {tuple(topk_ids.shape)}")
    if not 1 <= n_experts <= ROUTE_MAX_EXPERTS:
        raise ValueError(f"n_experts={n_experts} must be in [1, {ROUTE_MAX_EXPERTS}]")
    ids = topk_ids.to(torch.int64)
    if ids.stride(-1) != 1:
        ids = ids.contiguous()
    T, k = ids.shape
    N = T * k
    if cap < 0:
        raise ValueError(f"cap={cap} must be >= 0")
    if slots is None:
        slots = route_slots(N, n_experts, cap)
    dev = ids.device
    eids = torch.empty(slots, dtype=torch.int32, device=dev)
    row_off = torch.empty(slots + 1, dtype=torch.int32, device=dev)
    order = torch.empty(max(N, 1), dtype=torch.int32, device=dev)
    pos = torch.empty(max(N, 1), dtype=torch.int32, device=dev)
    info = torch.empty(3, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        rc = _hiplib.load().gnf4_hip_route_groups(
            ids.data_ptr(), ids.stride(0), T, k, n_experts, slots, cap, eids.data_ptr(),
            row_off.data_ptr(), order.data_ptr(), pos.data_ptr(), info.data_ptr(),
            _stream_ptr(dev))
    _hiplib.check(rc, "route_groups")
    return RoutePlan(eids, row_off, order, pos, info, T, k, n_experts, slots, cap)


def gather_rows(x: torch.Tensor, plan: RoutePlan) -> torch.Tensor:
    """``x [T, K]`` bf16 rows in grouped order: ``out[r] = x[order[r] // k]``."""
    _dev_check(x, "gather_rows")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"gather_rows: x must be bfloat16, got {x.dtype}")
    T, K = x.shape
    if T != plan.T:
        raise ValueError(f"x has {T} rows, the plan {plan.T} tokens")
    if x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    out = torch.empty(plan.rows, K, dtype=torch.bfloat16, device=x.device)
    with torch.cuda.device(x.device):
        rc = _hiplib.load().gnf4_hip_gather_rows(
            x.data_ptr(), x.stride(0), plan.order.data_ptr(), plan.rows, plan.k, K,
            out.data_ptr(), out.stride(0), _stream_ptr(x.device))
    _hiplib.check(rc, "gather_rows")
    return out


def combine(y: torch.Tensor, plan: RoutePlan, topk_weights: torch.Tensor) -> torch.Tensor:
    """``out[t] = sum_j w[t, j] * y[pos[t * k + j]]`` in fp32, j ascending,
    one bf16 rounding: the unsort + weight + sum of the reference's MoE
    block (arena_moe_patch.py:59-65)."""
    _dev_check(y, "combine")
    if y.dtype != torch.bfloat16:
        raise TypeError(f"combine: y must be bfloat16, got {y.dtype}")
    N, D = y.shape
    if N != plan.rows:
        raise ValueError(f"y has {N} rows, the plan {plan.rows}")
    w = topk_weights.to(torch.bfloat16)
    if tuple(w.shape) != (plan.T, plan.k):
        raise ValueError(f"topk_weights {tuple(w.shape)} != {(plan.T, plan.k)}")
    if w.stride(-1) != 1:
        w = w.contiguous()
    if y.stride(-1) != 1 or y.stride(0) % 8 or y.data_ptr() % 16:
        y = y.contiguous()
    out = torch.empty(plan.T, D, dtype=torch.bfloat16, device=y.device)
    with torch.cuda.device(y.device):
        rc = _hiplib.load().gnf4_hip_route_combine(
            y.data_ptr(), y.stride(0), plan.pos.data_ptr(), w.data_ptr(), w.stride(0), plan.T,
            plan.k, D, out.data_ptr(), out.stride(0), _stream_ptr(y.device))
    _hiplib.check(rc, "combine")
    return out


def _decode_fwd(a, W, S, plan: RoutePlan, max_m: int):
    """Decode forward over the plan's device tables (no host read)."""
    E, N, _ = W.shape
    K = a.shape[1]
    W, S = _aligned_rows(W, 16), _scales_view(S)
    out = torch.empty(a.shape[0], N, dtype=torch.bfloat16, device=a.device)
    with torch.cuda.device(a.device):
        rc = _hiplib.load().gnf4_hip_grouped_decode_routed(
            _hiplib.FMT_NF4, a.data_ptr(), _hiplib.DTYPE_BF16, a.stride(0),
            W.data_ptr(), W.stride(0), W.stride(1), S.data_ptr(), S.stride(0), S.stride(1),
            plan.eids.data_ptr(), plan.row_off.data_ptr(), plan.slots, max_m, N, K,
            out.data_ptr(), out.stride(0), _stream_ptr(a.device))
    _hiplib.check(rc, "moe_ffn")
    return out


def _route_decode(x, n_experts, k, topk_ids=None, logits=None, mode=0, norm=False,
                  cap=DECODE_GROUP_CAP):
    """The one-launch decode prologue (T <= 16): top-k (when ``logits`` is
    given), grouping (groups of at most ``cap`` rows) and gather. Returns
    (plan, gathered rows, ids, weights)."""
    T, K = x.shape
    dev = x.device
    N = T * k
    slots = route_slots(N, n_experts, cap)
    if logits is not None:
        lg = logits.float()
        if lg.stride(-1) != 1:
            lg = lg.contiguous()
        ids = torch.empty(T, k, dtype=torch.int64, device=dev)
        wts = torch.empty(T, k, dtype=torch.bfloat16, device=dev)
        lg_ptr, ld, w_ptr = lg.data_ptr(), lg.stride(0), wts.data_ptr()
    else:
        ids = topk_ids.to(torch.int64)
        if ids.stride(-1) != 1:
            ids = ids.contiguous()
        wts = None
        lg_ptr, ld, w_ptr = None, 0, None
    plan = RoutePlan(torch.empty(slots, dtype=torch.int32, device=dev),
                     torch.empty(slots + 1, dtype=torch.int32, device=dev),
                     torch.empty(max(N, 1), dtype=torch.int32, device=dev),
                     torch.empty(max(N, 1), dtype=torch.int32, device=dev),
                     torch.empty(3, dtype=torch.int32, device=dev), T, k, n_experts, slots, cap)
    a = torch.empty(N, K, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        rc = _hiplib.load().gnf4_hip_route_decode(
            lg_ptr, ld, T, n_experts, k, mode, int(bool(norm)), ids.data_ptr(), ids.stride(0),
            w_ptr, k, x.data_ptr(), x.stride(0), K, slots, cap, plan.eids.data_ptr(),
            plan.row_off.data_ptr(), plan.order.data_ptr(), plan.pos.data_ptr(),
            plan.info.data_ptr(), a.data_ptr(), a.stride(0), _stream_ptr(dev))
    _hiplib.check(rc, "route_decode")
    return plan, a, ids, wts


def moe_layer(x, router_logits, k, gu_packed, gu_absmax, dn_packed, dn_absmax, mode=0,
              norm=False, fused: bool | None = None):
    """A whole MoE expert layer from router logits: top-k (``route_topk``
    semantics) -> grouping -> gather -> expert FFN -> combine. Returns
    ``(out [T, D] bf16, topk_ids, topk_weights)``. At decode (T <= 16) the
    routing prologue is one launch and nothing is read on the host."""
    _dev_check(x, "moe_layer")
    T = x.shape[0]
    if router_logits.dim() != 2 or router_logits.shape[0] != T:
        raise ValueError(f"router_logits {tuple(router_logits.shape)} does not match {T} tokens")
    nf4_ffn._check_shapes(x, gu_packed, gu_absmax, dn_packed, dn_absmax)
    if T <= DECODE_MAX_ROWS and gu_packed.shape[0] <= ROUTE_MAX_EXPERTS:
        if not (1 <= k <= min(router_logits.shape[1], ROUTE_MAX_K)):
            raise ValueError(f"k={k} must be in [1, min(E, {ROUTE_MAX_K})]")
        if mode not in (0, 1):
            raise ValueError(f"mode must be 0 or 1, got {mode}")
        xb = nf4_grouped._bf16_activations(x, "moe_layer")
        plan, a, ids, wts = _route_decode(xb, gu_packed.shape[0], k, logits=router_logits,
                                          mode=mode, norm=norm)
        y = _expert_ffn_decode(a, plan, gu_packed, gu_absmax, dn_packed, dn_absmax, fused)
        return combine(y, plan, wts), ids, wts
    ids, wts = route_topk(router_logits, k, mode, norm)
    return moe_ffn(x, ids, wts, gu_packed, gu_absmax, dn_packed, dn_absmax, fused), ids, wts


def _expert_ffn_decode(a, plan, gu_packed, gu_absmax, dn_packed, dn_absmax, fused):
    H, n_dn = gu_packed.shape[1] // 2, dn_packed.shape[1]
    max_m = max(plan.max_rows_bound(), 1)
    if fused is None:
        fused = nf4_ffn._auto_fused(plan.slots, max_m, a.shape[1], H, n_dn)
    if fused:
        return nf4_ffn._launch_fused(a, gu_packed, gu_absmax, dn_packed, dn_absmax, plan.eids,
                                     plan.row_off, plan.slots, max_m)
    h = nf4_ffn.silu_mul_locked(_decode_fwd(a, gu_packed, gu_absmax, plan, max_m))
    return _decode_fwd(h, dn_packed, dn_absmax, plan, max_m)


def moe_ffn(x, topk_ids, topk_weights, gu_packed, gu_absmax, dn_packed, dn_absmax,
            fused: bool | None = None):
    """One MoE expert layer: ``sum_j w[t, j] * FFN_{e(t, j)}(x[t])`` with the
    grouped NF4 expert FFN (gate_up -> silu(gate) * up -> down).

    ``x [T, K]`` bf16; ``topk_ids [T, k]`` and ``topk_weights [T, k]`` on the
    device (from ``route_topk`` or the model's own router). With T <= 16
    (decode) nothing is read on the host: the routing tables stay on the
    device and the expert FFN runs as the fused call (two GEMV launches for
    T <= 4 at 1024 < K <= 2048 and T <= 2 at K <= 1024, one launch
    otherwise; above
    ``nf4_ffn.FUSED_MAX_UNITS`` workgroup units of that launch, decode
    forward -> silu-multiply -> decode forward), so the layer can be
    graph-captured.
    Larger T reads the group sizes once and takes the tiled kernels."""
    _dev_check(x, "moe_ffn")
    T, K = x.shape
    E = gu_packed.shape[0]
    H, n_dn = gu_packed.shape[1] // 2, dn_packed.shape[1]
    nf4_ffn._check_shapes(x, gu_packed, gu_absmax, dn_packed, dn_absmax)
    if topk_ids.dim() != 2 or topk_ids.shape[0] != T:
        raise ValueError(f"topk_ids {tuple(topk_ids.shape)} does not match {T} tokens")
    xb = nf4_grouped._bf16_activations(x, "moe_ffn")
    if T <= DECODE_MAX_ROWS and E <= ROUTE_MAX_EXPERTS:
        plan, a, _ids, _w = _route_decode(xb, E, topk_ids.shape[1], topk_ids=topk_ids)
        y = _expert_ffn_decode(a, plan, gu_packed, gu_absmax, dn_packed, dn_absmax, fused)
    else:
        plan = route_groups(topk_ids, E)
        a = gather_rows(xb, plan)
        sizes, ids = plan.host_groups()
        y = nf4_ffn.gemm_nf4_ffn_grouped(a, gu_packed, gu_absmax, dn_packed, dn_absmax, sizes,
                                         ids, fused=False if fused is None else fused)
    return combine(y, plan, topk_weights)
