// gnf4_route.hip -- device-side MoE routing around the grouped 4-bit expert
// GEMM on MI355X (gfx950): top-k selection with softmax weights, grouping of
// (token, slot) rows by expert, the gather of activations into group order,
// and the weighted combine back to token order.
//
// With these, a decode MoE layer (router logits -> top-k -> grouped expert
// FFN -> combine) runs on the device end to end: no host reads of the
// routing, so a whole layer can be captured in one HIP graph.
//
// Reference behaviour followed:
//   * top-k + softmax weights: gnf4_route_epilogue_bf16,
//     gnf4_native/cpu_kernels.c:1408-1471 (selection = stable descending sort,
//     ties to the lower index; mode 0 softmax over all logits gathered at the
//     selection, optionally renormalised; mode 1 softmax over the selected
//     logits; weights rounded to bf16 nearest-even);
//   * grouping, gather and combine: the sort / count / unsort around the
//     expert matmuls in kernel/arena_moe_patch.py:41-66 (tokens grouped by
//     expert in ascending expert order, rows of one expert in (token, slot)
//     order; output = sum over slots of weight * expert output).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gnf4_hip.h"

namespace {

typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;

constexpr int kRouteMaxK = 64;        // as the reference's epilogue (bv[64])
constexpr int kRouteMaxPerLane = 16;  // E <= 1024
constexpr int kGroupThreads = 1024;
constexpr int kGroupWaves = kGroupThreads / 64;
constexpr int kGroupMaxE = 512;

__device__ __forceinline__ uint16_t bf16_rne(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// Wave-wide reductions on the DPP network: xor-1 and xor-2 quad
// permutes, the half-row and row mirrors, then row broadcasts 15 and 31
// carry each row's result into the next rows; lane 63 ends with the whole
// wave's value, which readlane makes uniform. A fixed sequence, so sums are
// bitwise reproducible.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140,
              kDppBcast15 = 0x142, kDppBcast31 = 0x143;

template <class Op>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v, uint32_t identity, Op op) {
  const int x = (int)v, id = (int)identity;
  int t;
  t = __builtin_amdgcn_update_dpp(id, x, kDppXor1, 0xF, 0xF, false);
  v = op(v, (uint32_t)t);
  t = __builtin_amdgcn_update_dpp(id, (int)v, kDppXor2, 0xF, 0xF, false);
  v = op(v, (uint32_t)t);
  t = __builtin_amdgcn_update_dpp(id, (int)v, kDppHalfMirror, 0xF, 0xF, false);
  v = op(v, (uint32_t)t);
  t = __builtin_amdgcn_update_dpp(id, (int)v, kDppMirror, 0xF, 0xF, false);
  v = op(v, (uint32_t)t);
  t = __builtin_amdgcn_update_dpp(id, (int)v, kDppBcast15, 0xA, 0xF, false);
  v = op(v, (uint32_t)t);
  t = __builtin_amdgcn_update_dpp(id, (int)v, kDppBcast31, 0xC, 0xF, false);
  v = op(v, (uint32_t)t);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return wave_reduce_u32(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return wave_reduce_u32(v, 0xFFFFFFFFu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}

__device__ __forceinline__ float wave_sum(float x) {
  const uint32_t r = wave_reduce_u32(__float_as_uint(x), 0u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  });
  return __uint_as_float(r);
}

// Order-preserving map of a float to u32 (larger float -> larger key; -0
// and +0 share a key, as they compare equal). Key 0 is below every non-NaN
// value's key and marks "no candidate".
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u << 1) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Top-k of one token's logits by one wave. Lane l holds logits l, l + 64,
// ...; each of the k rounds takes the wave's largest remaining key (DPP max),
// then the lowest expert index holding it (DPP min): the stable descending
// order. Lane j < k returns the j-th pick and its weight.
template <int kPerLane>
__device__ __forceinline__ void topk_token(const float* __restrict__ lg, int E, int k, int mode,
                                           int norm, int lane, int& sel_i, float& w) {
  float v[kPerLane];
  uint32_t key[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? lg[e] : 0.0f;
    key[i] = e < E ? order_key(v[i]) : 0u;
  }
  // every non-NaN logit has a nonzero key (NaN logits are unspecified input)
  float sel_v = 0.0f;
  sel_i = 0;
  for (int j = 0; j < k; ++j) {
    uint32_t best = 0u;
    int best_e = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i)   // ascending e: strict > keeps the lower index
      if (key[i] > best) {
        best = key[i];
        best_e = lane + 64 * i;
      }
    const uint32_t top = wave_max_u32(best);
    const int pick = (int)wave_min_u32(best == top ? (uint32_t)best_e : 0xFFFFFFFFu);
    float picked = 0.0f;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i)
      if (lane + 64 * i == pick) {
        picked = v[i];
        key[i] = 0u;
      }
    // the owner lane (pick % 64) holds the value; broadcast it
    picked = __uint_as_float((uint32_t)__builtin_amdgcn_readlane(
        (int)__float_as_uint(picked), pick & 63));
    if (lane == j) {
      sel_v = picked;
      sel_i = pick;
    }
  }
  const bool mine = lane < k;
  if (mode == 0) {
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < kPerLane; ++i)
      if (lane + 64 * i < E) m = fmaxf(m, v[i]);
    m = __uint_as_float(wave_reduce_u32(__float_as_uint(m), __float_as_uint(-__builtin_inff()),
                                        [](uint32_t a, uint32_t b) {
                                          return __float_as_uint(fmaxf(__uint_as_float(a),
                                                                       __uint_as_float(b)));
                                        }));
    float z = 0.0f;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i)
      if (lane + 64 * i < E) z += expf(v[i] - m);
    z = wave_sum(z);
    w = mine ? expf(sel_v - m) / z : 0.0f;
    if (norm) w = w / wave_sum(w);
  } else {
    const float m = __uint_as_float((uint32_t)__builtin_amdgcn_readlane(
        (int)__float_as_uint(sel_v), 0));
    const float ex = mine ? expf(sel_v - m) : 0.0f;
    w = ex / wave_sum(ex);
  }
}

template <int kPerLane>
__global__ void __launch_bounds__(256) k_route_topk(const float* __restrict__ logits, int64_t ld,
                                                    int64_t T, int E, int k, int mode, int norm,
                                                    int64_t* __restrict__ idx,
                                                    int64_t idx_stride,
                                                    uint16_t* __restrict__ wts,
                                                    int64_t wts_stride) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;   // uniform per wave
  int sel_i;
  float w;
  topk_token<kPerLane>(logits + t * ld, E, k, mode, norm, lane, sel_i, w);
  if (lane < k) {
    idx[t * idx_stride + lane] = sel_i;
    wts[t * wts_stride + lane] = bf16_rne(w);
  }
}

// Grouping of N = T * k rows (row i = token i / k, slot i % k) by expert, in
// one workgroup of 16 waves. Wave w owns the contiguous rows
// [w * S, (w + 1) * S). (1) per-wave expert counts in LDS; (2) per expert, the
// waves' exclusive offsets and the expert total; (3) a scan over experts:
// active experts get consecutive group numbers in ascending expert order;
// (4) each wave walks its rows in order, 64 at a time, and places the rows of
// one expert at once (ballot), so rows of an expert stay in row order.
//
// Outputs: eids[g], row_off[g] for g < slots (groups past the active count
// are empty: row_off = N, eids = 0), row_off[slots] = N; order[r] = the row
// placed at grouped position r (-1 for the positions past the valid rows,
// as many as out-of-range ids); pos[i] = grouped position of row i (-1 for
// an out-of-range expert id, which is also flagged in info[2]); info[0] =
// active groups, info[1] = the largest group.
// cap > 0: an expert's rows form groups of at most cap rows (consecutive
// groups, the same expert id), so no group is larger than cap.
// `order_lds`, when not null, receives a copy of `order` in LDS.
// Groups of an expert with c rows: 0, 1, or ceil(c / cap) when capped.
__device__ __forceinline__ int groups_of(int c, int cap) {
  return c <= 0 ? 0 : cap > 0 ? (c + cap - 1) / cap : 1;
}

__device__ __forceinline__ void group_rows(const int64_t* ids, int64_t ids_stride, int64_t T,
                                           int k, int E, int slots, int cap,
                                           int32_t* __restrict__ eids,
                                           int32_t* __restrict__ row_off,
                                           int32_t* __restrict__ order,
                                           int32_t* __restrict__ pos,
                                           int32_t* __restrict__ info,
                                           int32_t* order_lds = nullptr,
                                           bool writer = true) {
  __shared__ int32_t s_cnt[kGroupWaves][kGroupMaxE];   // per-wave counts, then cursors
  __shared__ int32_t s_base[kGroupMaxE];              // first grouped position of expert e
  __shared__ int32_t s_scan[kGroupThreads];
  __shared__ int32_t s_scan2[kGroupThreads];
  __shared__ int32_t s_max, s_bad;
  // row indices fit in 32 bits (the host checks T * k < 2^31)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = (int)(T * k);
  const int S = (N + kGroupWaves - 1) / kGroupWaves;
  const int r0 = wave * S, r1 = r0 + S < N ? r0 + S : N;
  for (int i = tid; i < kGroupWaves * kGroupMaxE; i += kGroupThreads) (&s_cnt[0][0])[i] = 0;
  if (tid == 0) {
    s_max = 0;
    s_bad = 0;
  }
  __syncthreads();
  // (1) counts
  for (int i = r0 + lane; i < r1; i += 64) {
    const int64_t e = ids[(int64_t)(i / k) * ids_stride + i % k];
    if (e >= 0 && e < E)
      atomicAdd(&s_cnt[wave][e], 1);
    else
      s_bad = 1;
  }
  __syncthreads();
  // (2) per expert: exclusive offsets over waves, totals
  int tot = 0;
  if (tid < E) {
    for (int w = 0; w < kGroupWaves; ++w) {
      const int c = s_cnt[w][tid];
      s_cnt[w][tid] = tot;
      tot += c;
    }
  }
  // (3) inclusive scans of totals and of the active flag over experts
  s_scan[tid] = tid < E ? tot : 0;
  s_scan2[tid] = tid < E ? groups_of(tot, cap) : 0;
  __syncthreads();
  for (int off = 1; off < kGroupThreads; off <<= 1) {
    const int a = tid >= off ? s_scan[tid - off] : 0;
    const int b = tid >= off ? s_scan2[tid - off] : 0;
    __syncthreads();
    s_scan[tid] += a;
    s_scan2[tid] += b;
    __syncthreads();
  }
  if (tid < E) {
    const int base = s_scan[tid] - tot;
    s_base[tid] = base;
    if (tot > 0) {
      const int ng = groups_of(tot, cap);
      const int g = s_scan2[tid] - ng;
      for (int j = 0; writer && j < ng && g + j < slots; ++j) {
        eids[g + j] = tid;
        row_off[g + j] = base + j * cap;
      }
      atomicMax(&s_max, cap > 0 && tot > cap ? cap : tot);
    }
  }
  const int active = s_scan2[kGroupThreads - 1];
  for (int g = active + tid; writer && g < slots; g += kGroupThreads) {
    eids[g] = 0;
    row_off[g] = (int32_t)N;
  }
  // rows of out-of-range ids have no grouped position: the positions past
  // the valid rows hold -1 (their gathered rows are zero)
  for (int r = s_scan[kGroupThreads - 1] + tid; r < N; r += kGroupThreads) {
    if (writer) order[r] = -1;
    if (order_lds) order_lds[r] = -1;
  }
  __syncthreads();   // every wave's atomicMax on s_max has landed
  if (writer && tid == 0) {
    row_off[slots] = (int32_t)N;
    info[0] = active;
    info[1] = s_max;
    info[2] = s_bad;
  }
  // (4) stable placement, 64 rows at a time per wave
  for (int c0 = r0; c0 < r1; c0 += 64) {
    const int i = c0 + lane;
    const bool valid = i < r1;
    int64_t e = valid ? ids[(int64_t)(i / k) * ids_stride + i % k] : -1;
    const bool ok = valid && e >= 0 && e < E;
    if (writer && valid && !ok) pos[i] = -1;
    uint64_t pending = __builtin_amdgcn_ballot_w64(ok);
    while (pending) {
      const int leader = __builtin_ctzll(pending);
      const int le = __shfl((int)e, leader, 64);
      const uint64_t mask = __builtin_amdgcn_ballot_w64(ok && e == le);
      const int cur = s_cnt[wave][le];
      if (ok && e == le) {
        const int rank = __builtin_popcountll(mask & ((1ull << lane) - 1ull));
        const int p = s_base[le] + cur + rank;
        if (writer) {
          order[p] = (int32_t)i;
          pos[i] = p;
        }
        if (order_lds) order_lds[p] = (int32_t)i;
      }
      if (lane == leader) s_cnt[wave][le] = cur + __builtin_popcountll(mask);
      pending &= ~mask;
    }
  }
}

__global__ void __launch_bounds__(kGroupThreads) k_route_groups(
    const int64_t* __restrict__ ids, int64_t ids_stride, int64_t T, int k, int E, int slots,
    int cap, int32_t* __restrict__ eids, int32_t* __restrict__ row_off,
    int32_t* __restrict__ order, int32_t* __restrict__ pos, int32_t* __restrict__ info) {
  group_rows(ids, ids_stride, T, k, E, slots, cap, eids, row_off, order, pos, info);
}

// group_rows' outputs computed by one wave (the calling wave, all 64 lanes)
// for at most 64 rows (N = T * k <= 64: the decode prologue at a few
// tokens), with no workgroup barrier. Counts by LDS atomics into s_cnt[E];
// the exclusive scans over experts run across the lanes (lane l owns
// experts [l P, l P + P), P = ceil(E / 64)) with shuffles; lane i places row
// i after the earlier rows of its expert. Same outputs, bit for bit. `ids`
// is the row-major [T, k] array (row i at ids[i]).
__device__ __forceinline__ void group_rows_wave(const int64_t* ids, int64_t T, int k, int E,
                                                int slots, int cap, int32_t* __restrict__ eids,
                                                int32_t* __restrict__ row_off,
                                                int32_t* __restrict__ order,
                                                int32_t* __restrict__ pos,
                                                int32_t* __restrict__ info, int32_t* order_lds,
                                                int32_t* s_cnt, int32_t* s_base, bool writer) {
  const int lane = threadIdx.x & 63;
  const int N = (int)(T * k);
  for (int e = lane; e < E; e += 64) s_cnt[e] = 0;
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the zeros before the counts
  int bad = 0;
  for (int i = lane; i < N; i += 64) {
    const int64_t e = ids[i];
    if (e >= 0 && e < E)
      atomicAdd(&s_cnt[e], 1);
    else
      bad = 1;
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
  // the lane's experts: totals and active counts, then exclusive scans
  constexpr int kMaxP = kGroupMaxE / 64;
  const int P = (E + 63) / 64;
  int c[kMaxP];
  int tot = 0, act = 0, mx = 0;
#pragma unroll
  for (int j = 0; j < kMaxP; ++j) {
    const int e = lane * P + j;
    c[j] = j < P && e < E ? s_cnt[e] : 0;
    tot += c[j];
    act += groups_of(c[j], cap);
    const int cm = cap > 0 && c[j] > cap ? cap : c[j];
    mx = cm > mx ? cm : mx;
  }
  int tot_x = tot, act_x = act;   // inclusive scans over lanes
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t1 = __shfl_up(tot_x, d, 64), a1 = __shfl_up(act_x, d, 64);
    if (lane >= d) {
      tot_x += t1;
      act_x += a1;
    }
  }
  int base = tot_x - tot, g = act_x - act;   // exclusive
#pragma unroll
  for (int j = 0; j < kMaxP; ++j) {
    const int e = lane * P + j;
    if (j < P && e < E) {
      s_base[e] = base;
      const int ng = groups_of(c[j], cap);
      for (int t = 0; t < ng; ++t, ++g) {
        if (writer && g < slots) {
          eids[g] = e;
          row_off[g] = base + t * cap;
        }
      }
      base += c[j];
    }
  }
  const int active = __shfl(act_x, 63, 64);
  const int max_group = (int)wave_max_u32((uint32_t)mx);
  // positions past the valid rows (out-of-range ids) hold -1
  for (int r = __shfl(tot_x, 63, 64) + lane; r < N; r += 64) {
    if (writer) order[r] = -1;
    if (order_lds) order_lds[r] = -1;
  }
  for (int gg = active + lane; writer && gg < slots; gg += 64) {
    eids[gg] = 0;
    row_off[gg] = (int32_t)N;
  }
  if (writer && lane == 0) {
    row_off[slots] = (int32_t)N;
    info[0] = active;
    info[1] = max_group;
    info[2] = bad;
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);   // bases before the placement reads
  // stable placement: row i goes after the earlier rows of its expert, whose
  // number comes from a walk over the lanes' expert ids (no LDS round trip
  // per expert)
  const int i = lane;
  const bool valid = i < N;
  const int64_t e = valid ? ids[i] : -1;
  const bool ok = valid && e >= 0 && e < E;
  int rank = 0;
  for (int j = 0; j < N; ++j) {
    const int ej = __builtin_amdgcn_readlane((int)e, j);
    rank += (j < i && ej == (int)e) ? 1 : 0;
  }
  if (writer && valid && !ok) pos[i] = -1;
  if (ok) {
    const int p = s_base[e] + rank;
    if (writer) {
      order[p] = (int32_t)i;
      pos[i] = p;
    }
    if (order_lds) order_lds[p] = (int32_t)i;
  }
}

// The whole decode routing prologue in one workgroup (T <= 16 tokens):
// top-k of each token's logits by one wave (skipped when the caller passes
// its own ids: logits == nullptr), the grouping, and the activation rows in
// group order. The ids and the order stay in LDS between the phases. Where
// x fits kDecodeHold 16-byte pieces per thread, it is loaded into registers
// at the start (its loads overlap the logits' and the top-k), and after the
// grouping each piece is stored to its token's k grouped positions: no load
// waits on the grouping. Otherwise the rows are gathered after the grouping,
// eight 16-byte loads in flight per thread.
// The rows' stores (T * k rows of K, 512 KiB at 16 tokens x top-8 x 2048)
// are spread over the grid's workgroups: each repeats the top-k and the
// grouping in its own LDS (a few microseconds of latency, not of
// bandwidth), only workgroup 0 writes the ids, weights and tables, and
// workgroup b stores the rows of its slice of x. One workgroup alone is
// bound by one CU's store rate (16 tokens: 6.6 us for the stores).
constexpr int kDecodeMaxRows = kGroupWaves * kRouteMaxK;   // T * k <= 1024
constexpr int kDecodeHold = 8;

template <int kPerLane>
__global__ void __launch_bounds__(kGroupThreads) k_route_decode(
    const float* __restrict__ logits, int64_t ld, int64_t T, int E, int k, int mode, int norm,
    int64_t* idx, int64_t idx_stride, uint16_t* __restrict__ wts, int64_t wts_stride,
    const uint16_t* __restrict__ x, int64_t ldx, int64_t K, int slots, int cap,
    int32_t* __restrict__ eids, int32_t* __restrict__ row_off, int32_t* __restrict__ order,
    int32_t* __restrict__ pos, int32_t* __restrict__ info, uint16_t* __restrict__ a_out,
    int64_t lda) {
  __shared__ int64_t s_ids[kDecodeMaxRows];
  __shared__ int32_t s_order[kDecodeMaxRows];
  __shared__ int32_t s_pos[kDecodeMaxRows];
  __shared__ int32_t s_cnt1[kGroupMaxE], s_base1[kGroupMaxE];
  __shared__ int32_t s_valid;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwg = (int)gridDim.x, wg = (int)blockIdx.x;
  const bool writer = wg == 0;
  const int N = (int)(T * k);
  // 32-bit index math (the host checks T * k * K < 2^31)
  const int vec = (int)(K / 8);
  const int xtot = (int)T * vec;
  // this workgroup's slice of x's 16-byte pieces
  const int per = nwg == 1 ? xtot : (xtot + nwg - 1) / nwg;
  const int q_lo = wg * per, q_hi = q_lo + per < xtot ? q_lo + per : xtot;
  const bool hold = per <= kDecodeHold * kGroupThreads;   // uniform
  u32x4_t xv[kDecodeHold];
  if (hold) {
#pragma unroll
    for (int u = 0; u < kDecodeHold; ++u) {
      const int q = q_lo + threadIdx.x + u * kGroupThreads;
      if (q < q_hi) {
        const int t = q / vec, c = (q - t * vec) * 8;
        xv[u] = *reinterpret_cast<const u32x4_t*>(x + (int64_t)t * ldx + c);
      }
    }
  }
  if (logits) {
    if (wave < T) {
      int sel_i;
      float w;
      topk_token<kPerLane>(logits + wave * ld, E, k, mode, norm, lane, sel_i, w);
      if (lane < k) {
        if (writer) {
          idx[wave * idx_stride + lane] = sel_i;
          wts[wave * wts_stride + lane] = bf16_rne(w);
        }
        s_ids[wave * k + lane] = sel_i;
      }
    }
  } else {
    for (int i = threadIdx.x; i < N; i += kGroupThreads) s_ids[i] = idx[(i / k) * idx_stride + i % k];
  }
  __syncthreads();
  // the grouping: by one wave, with no workgroup barriers, for up to 64 rows
  if (N <= 64) {
    if (wave == 0)
      group_rows_wave(s_ids, T, k, E, slots, cap, eids, row_off, order, pos, info, s_order,
                      s_cnt1, s_base1, writer);
  } else {
    group_rows(s_ids, k, T, k, E, slots, cap, eids, row_off, order, pos, info, s_order, writer);
  }
  __syncthreads();
  if (hold) {
    // row i's grouped position (-1: an out-of-range id), and the first
    // position past the valid rows (the positions after it hold -1)
    if (threadIdx.x == 0) s_valid = N;
    for (int i = threadIdx.x; i < N; i += kGroupThreads) s_pos[i] = -1;
    __syncthreads();
    for (int p = threadIdx.x; p < N; p += kGroupThreads) {
      const int src = s_order[p];
      if (src >= 0)
        s_pos[src] = p;
      else
        atomicMin(&s_valid, p);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kDecodeHold; ++u) {
      const int q = q_lo + threadIdx.x + u * kGroupThreads;
      if (q < q_hi) {
        const int t = q / vec, c = (q - t * vec) * 8;
        for (int j = 0; j < k; ++j) {
          const int p = s_pos[t * k + j];
          if (p >= 0) *reinterpret_cast<u32x4_t*>(a_out + (int64_t)p * lda + c) = xv[u];
        }
      }
    }
    // positions past the valid rows gather nothing: zeros
    const int v = s_valid;
    for (int q = v * vec + wg * kGroupThreads + threadIdx.x; q < N * vec;
         q += nwg * kGroupThreads) {
      const int r = q / vec, c = (q - r * vec) * 8;
      *reinterpret_cast<u32x4_t*>(a_out + (int64_t)r * lda + c) = u32x4_t{0u, 0u, 0u, 0u};
    }
    return;
  }
  const int total = N * vec;
  constexpr int kInFlight = 8;
  for (int q0 = wg * kInFlight * kGroupThreads + threadIdx.x; q0 < total;
       q0 += nwg * kInFlight * kGroupThreads) {
    u32x4_t v[kInFlight];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      const int q = q0 + u * kGroupThreads;
      if (q < total) {
        const int r = q / vec, c = (q - r * vec) * 8;
        const int src = s_order[r];   // -1: no row (an out-of-range id)
        v[u] = src >= 0 ? *reinterpret_cast<const u32x4_t*>(x + (int64_t)(src / k) * ldx + c)
                        : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      const int q = q0 + u * kGroupThreads;
      if (q < total) {
        const int r = q / vec, c = (q - r * vec) * 8;
        *reinterpret_cast<u32x4_t*>(a_out + (int64_t)r * lda + c) = v[u];
      }
    }
  }
}

// out[r, :] = x[order[r] / k, :] for r < N (zeros where order[r] < 0). Eight
// bf16 per thread. Idx is
// uint32_t whenever N * K / 8 < 2^32 (64-bit division is a long software
// sequence on this GPU).
template <class Idx>
__global__ void __launch_bounds__(256) k_gather_rows(const uint16_t* __restrict__ x, int64_t ldx,
                                                     const int32_t* __restrict__ order, Idx N,
                                                     int k, Idx K, uint16_t* __restrict__ out,
                                                     int64_t ldo) {
  const Idx vec = K / 8, total = N * vec;
  for (Idx q = (Idx)blockIdx.x * blockDim.x + threadIdx.x; q < total;
       q += (Idx)gridDim.x * blockDim.x) {
    const Idx r = q / vec, c = (q - r * vec) * 8;
    const int32_t o = order[r];   // -1: no row (an out-of-range id), zeros
    *reinterpret_cast<u32x4_t*>(out + (int64_t)r * ldo + c) =
        o >= 0 ? *reinterpret_cast<const u32x4_t*>(x + (int64_t)(o / k) * ldx + c)
               : u32x4_t{0u, 0u, 0u, 0u};
  }
}

// out[t, d] = bf16(sum_j w[t, j] * y[pos[t * k + j], d]), j ascending, fp32.
// Rows with pos < 0 (an out-of-range expert id) contribute nothing. Slots go
// eight at a time: their positions and weights, then their rows, are loaded
// before any is used.
template <class Idx>
__global__ void __launch_bounds__(256) k_route_combine(const uint16_t* __restrict__ y, int64_t ldy,
                                                       const int32_t* __restrict__ pos,
                                                       const uint16_t* __restrict__ wts,
                                                       int64_t wts_stride, Idx T, int k, Idx D,
                                                       uint16_t* __restrict__ out, int64_t ldo) {
  const Idx vec = D / 8, total = T * vec;
  for (Idx q = (Idx)blockIdx.x * blockDim.x + threadIdx.x; q < total;
       q += (Idx)gridDim.x * blockDim.x) {
    const int64_t t = q / vec, c = (q - (Idx)t * vec) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < k; j0 += 8) {
      int32_t p[8];
      float w[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = j0 + jj;
        p[jj] = j < k ? pos[t * k + j] : -1;
        w[jj] = j < k ? bf16_to_f32(wts[t * wts_stride + j]) : 0.0f;
      }
      u32x4_t v[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
        v[jj] = p[jj] >= 0 ? *reinterpret_cast<const u32x4_t*>(y + (int64_t)p[jj] * ldy + c)
                           : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        if (p[jj] < 0) continue;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          acc[2 * h] += w[jj] * __uint_as_float(v[jj][h] << 16);
          acc[2 * h + 1] += w[jj] * __uint_as_float(v[jj][h] & 0xFFFF0000u);
        }
      }
    }
    u32x4_t o;
#pragma unroll
    for (int h = 0; h < 4; ++h)
      o[h] = (uint32_t)bf16_rne(acc[2 * h]) | ((uint32_t)bf16_rne(acc[2 * h + 1]) << 16);
    *reinterpret_cast<u32x4_t*>(out + t * ldo + c) = o;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int64_t grid_for(int64_t work_items, int threads) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return -1;
  const int64_t need = (work_items + threads - 1) / threads;
  const int64_t cap = (int64_t)cus * 8;
  return need < 1 ? 1 : (need < cap ? need : cap);
}

}  // namespace

extern "C" {

int gnf4_hip_route_topk(const float* logits, int64_t T, int64_t E, int64_t ld, int k, int mode,
                        int norm, int64_t* idx, int64_t idx_stride, uint16_t* wts,
                        int64_t wts_stride, void* stream) {
  if (T < 0 || E <= 0 || E > 64 * kRouteMaxPerLane || ld < E || k < 1 || k > kRouteMaxK ||
      k > E || (mode != 0 && mode != 1) || idx_stride < k || wts_stride < k)
    return -1;
  if (T == 0) return 0;
  if (!logits || !idx || !wts) return -1;
  const int64_t blocks = (T + 3) / 4;
  if (blocks > 0x7FFFFFFF) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int per_lane = (int)((E + 63) / 64);
#define GNF4_TOPK(P)                                                                        \
  hipLaunchKernelGGL((k_route_topk<P>), dim3((unsigned)blocks), dim3(256), 0, s, logits, ld, \
                     T, (int)E, k, mode, norm, idx, idx_stride, wts, wts_stride)
  if (per_lane <= 1)
    GNF4_TOPK(1);
  else if (per_lane <= 2)
    GNF4_TOPK(2);
  else if (per_lane <= 4)
    GNF4_TOPK(4);
  else if (per_lane <= 8)
    GNF4_TOPK(8);
  else
    GNF4_TOPK(16);
#undef GNF4_TOPK
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_route_groups(const int64_t* topk_ids, int64_t ids_stride, int64_t T, int k,
                          int64_t E, int slots, int cap, int32_t* eids, int32_t* row_off,
                          int32_t* order, int32_t* pos, int32_t* info, void* stream) {
  if (T < 0 || k < 1 || ids_stride < k || E <= 0 || E > kGroupMaxE || slots < 0 || cap < 0)
    return -1;
  if (T * k > 0x7FFFFFFF) return -1;
  if (!topk_ids || !eids || !row_off || !order || !pos || !info) return -1;
  hipLaunchKernelGGL(k_route_groups, dim3(1), dim3(kGroupThreads), 0,
                     static_cast<hipStream_t>(stream), topk_ids, ids_stride, T, k, (int)E,
                     slots, cap, eids, row_off, order, pos, info);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_route_decode(const float* logits, int64_t ld, int64_t T, int64_t E, int k,
                          int mode, int norm, int64_t* idx, int64_t idx_stride, uint16_t* wts,
                          int64_t wts_stride, const void* x, int64_t ldx, int64_t K, int slots,
                          int cap, int32_t* eids, int32_t* row_off, int32_t* order, int32_t* pos,
                          int32_t* info, void* a_out, int64_t lda, void* stream) {
  if (T < 0 || T > kGroupWaves || E <= 0 || E > kGroupMaxE || k < 1 || k > kRouteMaxK ||
      k > E || idx_stride < k || slots < 0 || cap < 0 || K <= 0 || K % 8 || ldx < K || ldx % 8 ||
      lda < K || lda % 8)
    return -1;
  if (logits && (ld < E || (mode != 0 && mode != 1) || !wts || wts_stride < k)) return -1;
  if (T * k * K >= 0x7FFFFFFF) return -1;   // the gather's 32-bit index math
  if (!idx || !x || !eids || !row_off || !order || !pos || !info || !a_out || !aligned16(x) ||
      !aligned16(a_out))
    return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int per_lane = (int)((E + 63) / 64);
  // about 32 KiB of grouped rows per workgroup (one at a token), at most 32
  int64_t nwg = (T * k * K * 2 + 32767) / 32768;
  nwg = nwg < 1 ? 1 : nwg > 32 ? 32 : nwg;
#define GNF4_PRO(P)                                                                           \
  hipLaunchKernelGGL((k_route_decode<P>), dim3((unsigned)nwg), dim3(kGroupThreads), 0, s,     \
                     logits, ld, T,                                                           \
                     (int)E, k, mode, norm, idx, idx_stride, wts, wts_stride,                  \
                     static_cast<const uint16_t*>(x), ldx, K, slots, cap, eids, row_off, order, \
                     pos, info, static_cast<uint16_t*>(a_out), lda)
  if (per_lane <= 1)
    GNF4_PRO(1);
  else if (per_lane <= 2)
    GNF4_PRO(2);
  else if (per_lane <= 4)
    GNF4_PRO(4);
  else
    GNF4_PRO(8);
#undef GNF4_PRO
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_gather_rows(const void* x, int64_t ldx, const int32_t* order, int64_t N, int k,
                         int64_t K, void* out, int64_t ldo, void* stream) {
  if (N < 0 || k < 1 || K <= 0 || K % 8 || ldx < K || ldx % 8 || ldo < K || ldo % 8) return -1;
  if (N == 0) return 0;
  if (!x || !order || !out || !aligned16(x) || !aligned16(out)) return -1;
  const int64_t grid = grid_for(N * (K / 8), 256);
  if (grid < 0) return -2;
  if (N * (K / 8) < (int64_t)0xFFFFFFFF)
    hipLaunchKernelGGL((k_gather_rows<uint32_t>), dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), ldx,
                       order, (uint32_t)N, k, (uint32_t)K, static_cast<uint16_t*>(out), ldo);
  else
    hipLaunchKernelGGL((k_gather_rows<int64_t>), dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), ldx,
                       order, N, k, K, static_cast<uint16_t*>(out), ldo);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_route_combine(const void* y, int64_t ldy, const int32_t* pos, const uint16_t* wts,
                           int64_t wts_stride, int64_t T, int k, int64_t D, void* out,
                           int64_t ldo, void* stream) {
  if (T < 0 || k < 1 || wts_stride < k || D <= 0 || D % 8 || ldy < D || ldy % 8 || ldo < D ||
      ldo % 8)
    return -1;
  if (T == 0) return 0;
  if (!y || !pos || !wts || !out || !aligned16(y) || !aligned16(out)) return -1;
  const int64_t grid = grid_for(T * (D / 8), 256);
  if (grid < 0) return -2;
  if (T * (D / 8) < (int64_t)0xFFFFFFFF)
    hipLaunchKernelGGL((k_route_combine<uint32_t>), dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(y), ldy,
                       pos, wts, wts_stride, (uint32_t)T, k, (uint32_t)D,
                       static_cast<uint16_t*>(out), ldo);
  else
    hipLaunchKernelGGL((k_route_combine<int64_t>), dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(y), ldy,
                       pos, wts, wts_stride, T, k, D, static_cast<uint16_t*>(out), ldo);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
