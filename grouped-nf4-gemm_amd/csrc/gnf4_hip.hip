// gnf4_hip.hip -- grouped 4-bit (NF4 / MXFP4) MoE expert GEMM for CDNA4 (gfx950).
//
// Computes, for tokens grouped by expert, out[t, :] = a[t, :] . dequant(W[e(t)])^T
// (forward) and grad_a[t, :] = grad_out[t, :] . dequant(W[e(t)]) (dgrad), in one
// launch for all active experts, from the packed [E, N, K/2] uint8 weights.
//
// Weight decode, shared by every kernel here (reference semantics:
// kernel/nf4_grouped.py:910-929 and kernel/mxfp4_pack_ref.py:46-70):
//   NF4   byte j of a row holds elements 2j (high nibble) and 2j+1 (low
//         nibble); w = NF4[code] * absmax[n, k / 64] is formed in fp32 (one
//         rounding) and rounded once to bf16 (RNE). The LUT lookup is a
//         64 KiB LDS table indexed by the whole packed byte: entry (byte, lane)
//         holds the fp32 pair (NF4[byte >> 4], NF4[byte & 15]) in a column
//         private to lane % 32, so a wave's 64 lookups never share an LDS
//         bank. One v_perm_b32 forms the byte address (byte << 8 | lane*8).
//   MXFP4 byte j holds elements 2j (low nibble) and 2j+1 (high nibble);
//         v_cvt_scalef32_pk_bf16_fp4 converts a nibble pair and multiplies by
//         2^(e - 127) in one instruction. e2m1 x 2^s is exact in bf16.
// The decoded bf16 weights feed v_mfma_f32_16x16x32_bf16 with fp32
// accumulation and a single bf16 rounding of each output.
//
// MFMA 16x16x32 operand layout used throughout (lane l = 0..63):
//   A: row l % 16, 8 consecutive k of slice (l / 16)
//   B: col l % 16, 8 consecutive k of slice (l / 16)
//   D: rows 4 * (l / 16) + i (i = 0..3), col l % 16
// The k-slice assignment only has to agree between A and B.
//
// Kernels:
//   k_decode_fwd   groups of <= 16 rows (decode). One wave streams a 16-row
//                  weight tile straight from HBM through registers, 16 bytes
//                  per lane per 128-element chunk, with a prefetch ring; the
//                  group's <= 16 activation rows ride along as the MFMA A
//                  operand. One workgroup per unit (group, 16-row n-tile);
//                  its four waves split the K chunks and reduce through LDS.
//   k_gemm_fwd     large groups (prefill). BM x 128 output tiles over ragged
//                  groups from a host tile table; per 64-wide k-step the
//                  activation tile and the decoded weight tile are staged in
//                  LDS (double buffered) and consumed by 4 waves.
//   k_gemm_dgrad   grad_a = grad_out . W, contracting over N in fixed 64-wide
//                  steps (two MFMAs, ascending n) so the output bits do not
//                  depend on the output tiling. The weight tile is decoded
//                  from the same [E, N, K/2] layout and written to LDS
//                  transposed (k-major) for the MFMA B operand.
//
// Everything is stream-ordered on the caller's stream. No allocation, no
// host synchronisation. Return codes: 0 ok, -1 shape/argument violation,
// -2 launch error.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "../../include/gnf4_hip.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2_t;
typedef __attribute__((ext_vector_type(2))) int v2i32_t;

constexpr int kNF4 = GNF4_FMT_NF4;
constexpr int kMX = GNF4_FMT_MXFP4;

// NF4 codebook, reference kernel/nf4_grouped.py:53-70 (code 7 is exactly 0).
__constant__ float c_nf4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f,
};

// ---------------------------------------------------------------- decode --

// The NF4 pair table: 256 bytes x 32 lane columns x float2 = 64 KiB. Entry
// (byte, column) holds the fp32 pair (NF4[byte >> 4], NF4[byte & 15]) in the
// column of lane % 32, so the lanes one LDS pass serves read distinct banks.
// Declared first so it sits at LDS offset 0: one v_perm_b32 then forms the
// full address byte << 8 | (lane % 32) * 8.
constexpr int kPairEntries = 256 * 32;

// Codebook entry `lane % 16` in one register per lane. Kernels load it before
// any weight load: vector loads complete in order, so a codebook read issued
// after the weights would hold the table build until every weight landed.
__device__ __forceinline__ int nf4_lut_lane() {
  return __float_as_int(c_nf4[threadIdx.x & 15]);
}

__device__ __forceinline__ void init_pair_table(float2* tab, int lut) {
  // Thread t fills the columns of byte t % 256 (all 32 of them with 256
  // threads, half of them with 512), rotating the column order by byte so one store instruction
  // touches distinct banks. Entries come from the codebook register of lanes
  // 0..15 through ds_bpermute.
  const unsigned b = threadIdx.x & 255;
  const float hi = __int_as_float(__builtin_amdgcn_ds_bpermute((int)((b >> 4) << 2), lut));
  const float lo = __int_as_float(__builtin_amdgcn_ds_bpermute((int)((b & 15) << 2), lut));
  const float2 e = make_float2(hi, lo);
  // with 512 threads the second 256 fill the other half of the columns
  const int j0 = threadIdx.x < 256 ? 0 : 16;
  const int nj = blockDim.x > 256 ? 16 : 32;
  for (int j = 0; j < nj; ++j) tab[b * 32 + ((j0 + j + b) & 31)] = e;
}

// Codebook value c (0..15) from immediate constants (a select chain): no
// memory load, so a table built from it need not wait for any.
__device__ __forceinline__ float nf4_code_imm(unsigned c) {
  float r = -1.0f;
  r = c == 1 ? -0.6961928009986877f : r;
  r = c == 2 ? -0.5250730514526367f : r;
  r = c == 3 ? -0.39491748809814453f : r;
  r = c == 4 ? -0.28444138169288635f : r;
  r = c == 5 ? -0.18477343022823334f : r;
  r = c == 6 ? -0.09105003625154495f : r;
  r = c == 7 ? 0.0f : r;
  r = c == 8 ? 0.07958029955625534f : r;
  r = c == 9 ? 0.16093020141124725f : r;
  r = c == 10 ? 0.24611230194568634f : r;
  r = c == 11 ? 0.33791524171829224f : r;
  r = c == 12 ? 0.44070982933044434f : r;
  r = c == 13 ? 0.5626170039176941f : r;
  r = c == 14 ? 0.7229568362236023f : r;
  r = c == 15 ? 1.0f : r;
  return r;
}

// The pair table of init_pair_table (64 KiB at LDS offset 0, 32 lane
// columns) filled by 512 threads from nf4_code_imm: thread t fills 16
// columns of byte t % 256.
__device__ __forceinline__ void init_pair_table_imm(char* smem) {
  const unsigned b = threadIdx.x & 255;
  const float2 e = make_float2(nf4_code_imm(b >> 4), nf4_code_imm(b & 15));
  const int j0 = threadIdx.x < 256 ? 0 : 16;
  float2* tab = reinterpret_cast<float2*>(smem);
#pragma unroll
  for (int j = 0; j < 16; ++j) tab[b * 32 + ((j0 + j + b) & 31)] = e;
}

__device__ __forceinline__ unsigned bf16x2_bits(float lo, float hi) {
  bf16x2_t r = {(__bf16)lo, (__bf16)hi};  // v_cvt_pk_bf16_f32, RNE
  return __builtin_bit_cast(unsigned, r);
}

// 8 NF4 elements of one packed dword -> 4 dwords of bf16 pairs in k order.
// lane_off = (lane % 32) * 8: the lane's private column in the pair table.
__device__ __forceinline__ u32x4_t nf4_dword_to_bf16(const float2* tab, unsigned x,
                                                     unsigned lane_off, float s) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned addr = __builtin_amdgcn_perm(x, lane_off, 0x0C0C0000u | ((4u + i) << 8));
    const float2 p = *reinterpret_cast<const float2*>(reinterpret_cast<const char*>(tab) + addr);
    r[i] = bf16x2_bits(p.x * s, p.y * s);
  }
  return r;
}

// Same, with the table at an LDS address below 16 MiB whose bits 8..15 are
// zero: `base_lane` = table address | lane column, and the address of byte b
// is base_lane with b in bits 8..15 (one v_perm_b32). `lds0` points at LDS
// address 0.
__device__ __forceinline__ u32x4_t nf4_dword_to_bf16_at(const char* lds0, unsigned x,
                                                        unsigned base_lane, float s) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned addr = __builtin_amdgcn_perm(x, base_lane, 0x0C020000u | ((4u + i) << 8));
    const float2 p = *reinterpret_cast<const float2*>(lds0 + addr);
    r[i] = bf16x2_bits(p.x * s, p.y * s);
  }
  return r;
}

// ---- exact three-part NF4 codebook (decode kernels) ----
//
// Every fp32 codebook value v splits exactly into three bf16 values,
// v = hi + mid + lo: hi keeps the top 16 bits of v's pattern (sign, exponent,
// 7 mantissa bits), the remainder r = v - hi is exact with at most 16
// significant bits, mid keeps r's top 16 bits and lo = r - mid is exact with
// at most 8 significant bits. Three bf16 MFMAs over the parts therefore sum
// codebook values at full fp32 precision (each product of a bf16 activation
// and a bf16 part is exact in fp32), and absmax multiplies the 64-element
// block sum once, in fp32, as the reference's GEMV does
// (kernel/nf4_grouped.py:508-511).
//
// The split table: 256 bytes x 16 lane columns x 16 B = 64 KiB. Entry (byte,
// column) holds the bf16 pairs (part[byte >> 4], part[byte & 15]) of hi, mid
// and lo in dwords 0..2 (element 2j, the high nibble, in the low half), so
// one 16-byte LDS read decodes a byte into the three MFMA operand dwords.
// Column = lane % 16: the 16 lanes of one LDS pass read distinct banks.
constexpr int kSplitCols = 16;
constexpr int kSplitTabBytes = 256 * kSplitCols * 16;
static_assert(kSplitTabBytes == 8 * kPairEntries, "split and pair tables take the same LDS");

__device__ __forceinline__ void nf4_split_parts(int lut, unsigned& himid, unsigned& lo) {
  const unsigned u = (unsigned)lut;
  const unsigned h = u & 0xFFFF0000u;
  const float r = __uint_as_float(u) - __uint_as_float(h);          // exact
  const unsigned rm = __float_as_uint(r) & 0xFFFF0000u;
  const float l = r - __uint_as_float(rm);                           // exact
  himid = (h >> 16) | rm;                  // hi in the low half, mid in the high half
  lo = __float_as_uint(l) >> 16;
}

// Fill the split table from the codebook register of lanes 0..15 (see
// nf4_lut_lane). Thread t fills byte t % 256; with 512 threads each byte's
// 16 columns are split over two threads. Columns rotate with the byte so one
// store instruction touches distinct banks.
__device__ __forceinline__ void init_split_table(char* tab, int lut) {
  unsigned hm, lo;
  nf4_split_parts(lut, hm, lo);
  const unsigned b = threadIdx.x & 255;
  const unsigned hmh = __builtin_amdgcn_ds_bpermute((int)((b >> 4) << 2), (int)hm);
  const unsigned hml = __builtin_amdgcn_ds_bpermute((int)((b & 15) << 2), (int)hm);
  const unsigned loh = __builtin_amdgcn_ds_bpermute((int)((b >> 4) << 2), (int)lo);
  const unsigned lol = __builtin_amdgcn_ds_bpermute((int)((b & 15) << 2), (int)lo);
  const u32x4_t e = {(hmh & 0xFFFFu) | (hml << 16), (hmh >> 16) | (hml & 0xFFFF0000u),
                     loh | (lol << 16), 0u};
  const int nj = blockDim.x > 256 ? 8 : 16;
  const int j0 = threadIdx.x < 256 ? 0 : 8;
  for (int j = 0; j < nj; ++j)
    *reinterpret_cast<u32x4_t*>(tab + b * (kSplitCols * 16) + (((j0 + j + b) & 15) * 16)) = e;
}

// 16-byte LDS read at a byte address: no base pointer arithmetic around it.
typedef __attribute__((address_space(3))) const u32x4_t lds_u32x4_t;
__device__ __forceinline__ u32x4_t lds_read16(unsigned addr) {
  return *(lds_u32x4_t*)(size_t)addr;
}
// The three bf16 parts of the four bytes of w (lane column lane_off), as the
// hi, mid and lo MFMA operands. One 16-byte read per byte: three separate
// 4-byte reads per byte into the operand registers measured 1.85x slower
// (three times the LDS instructions, four lanes per bank), 12-byte reads
// 2-10 % slower.
__device__ __forceinline__ void split_lookup(unsigned w, unsigned lane_off, u32x4_t& hi,
                                             u32x4_t& mid, u32x4_t& lo) {
  u32x4_t d[4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
    d[b] = lds_read16(__builtin_amdgcn_perm(w, lane_off, 0x0C0C0000u | ((4u + b) << 8)));
  hi = u32x4_t{d[0][0], d[1][0], d[2][0], d[3][0]};
  mid = u32x4_t{d[0][1], d[1][1], d[2][1], d[3][1]};
  lo = u32x4_t{d[0][2], d[1][2], d[2][2], d[3][2]};
}
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((address_space(3))) const f32x2_t lds_f32x2_t;
__device__ __forceinline__ f32x2_t lds_read8f(unsigned addr) {
  return *(lds_f32x2_t*)(size_t)addr;
}

// 8 MXFP4 elements of one packed dword (low nibble first) -> 4 bf16 pairs.
__device__ __forceinline__ u32x4_t mx_dword_to_bf16(unsigned x, float s) {
  u32x4_t r;
  r[0] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, s, 0));
  r[1] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, s, 1));
  r[2] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, s, 2));
  r[3] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, s, 3));
  return r;
}

// e8m0 byte -> fp32 2^(e - 127): e = 0 is the subnormal 2^-127, e = 255 is
// +inf (so a 0xFF block decodes to +-inf, and zero codes to NaN, like an
// exp2-multiply decode; reference kernel/mxfp4_grouped.py:13-15).
__device__ __forceinline__ float e8m0_to_f32(unsigned e) {
  return __uint_as_float(e == 0 ? 0x00400000u : (e << 23));
}

// Calls fn(integral_constant<I>) for I = 0 .. S - 1 while it returns true.
template <int I, int S>
struct StepUnroll {
  template <class Fn>
  __device__ __forceinline__ static bool run(Fn& fn) {
    if (!fn(std::integral_constant<int, I>{})) return false;
    return StepUnroll<I + 1, S>::run(fn);
  }
};
template <int S>
struct StepUnroll<S, S> {
  template <class Fn>
  __device__ __forceinline__ static bool run(Fn&) { return true; }
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f32x4_t mfma(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Activation chunk (8 consecutive elements) as bf16 bits. fp16 inputs are
// rejected on the host before launch; the kernels take bf16.
__device__ __forceinline__ u32x4_t load_a8(const uint16_t* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

// ============================================================ decode fwd ==

struct FwdArgs {
  const uint16_t* a;        // [T, lda] bf16
  int64_t lda;
  const uint8_t* B;         // [E, N, K/2]
  int64_t sbe, sbn;         // bytes
  const void* S;            // absmax f32 [E, N, K/64] or e8m0 u8 [E, N, K/32]
  int64_t sse, ssn;         // elements
  const int32_t* eids;      // [G]
  const int32_t* row_off;   // [G + 1] (ro_shift 0), [2 G] (ro_shift 1), or
                            // null: group g is the single row g
  const int32_t* t_row0;    // [n_mtiles] (gemm path)
  const int32_t* t_rows;
  const int32_t* t_group;
  int n_mtiles;
  int G;
  int max_m;                // largest group (decode path)
  // decode path: group g's rows are [row_off[g << ro_shift],
  // row_off[(g << ro_shift) + 1]): ro_shift 0 reads the G + 1 prefix offsets,
  // 1 a (first, end) pair per group, so the groups may come in any order
  int ro_shift;
  int64_t N, K;
  uint16_t* out;            // [T, ldo] bf16
  int64_t ldo;
  // host only: group ids and row offsets to pass in the GEMV kernels'
  // arguments (GemvIds), or null (the kernels read eids / row_off)
  const struct GemvIds* ids_inline;
  // host only: the groups come from device routing and any of them may be
  // empty (the launch covers a bound of the active groups)
  int sparse_groups;
};

// The groups of a decode launch of at most kGemvIdsMax groups, in the GEMV
// kernels' arguments (n > 0): the kernel reads them from the kernarg
// segment it loads anyway, instead of a table in memory behind it (one
// dependent round trip before the first weight load). Entry y (grid row y)
// is a group: its expert id e[y] and rows[y] = first row << 8 | row count.
// The host lists the groups largest first, so the workgroups of the groups
// that take the most passes are dispatched first (every output row is
// computed on its own: the order changes no bits). has_ro: the caller gave
// row offsets (the multi-row GEMV needs them).
constexpr int kGemvIdsMax = 384;
constexpr int kGemvRowsMax = 1 << 23;   // first rows must fit in rows[y] >> 8
struct GemvIds {
  int32_t e[kGemvIdsMax];
  int32_t rows[kGemvIdsMax];
  int32_t n;
  int32_t has_ro;
};

constexpr int kOOB = (int)0x80000000;  // buffer offset past every resource: loads 0

// Buffer resources: raw loads through them are bounds-checked by the
// hardware, so a masked lane gets zeros without a branch (and the compiler
// keeps exact vmcnt counts for the prefetched loads).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes < 0x7FFFFFFF ? (int)bytes : 0x7FFFFFFF;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

__device__ __forceinline__ u32x4_t buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Cache-policy bits of a buffer access: kScopeDevice (sc1) makes the access
// coherent at device scope, across the XCDs' separate L2 caches, without any
// cache writeback or invalidate.
constexpr int kScopeDevice = 16;

template <int kAux>
__device__ __forceinline__ u32x4_t buf_load16_aux(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAux));
}

__device__ __forceinline__ unsigned buf_load1(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}

// off | 0x80000000 when !ok, through an opaque VALU op so the compiler cannot
// turn the masked load back into a branch around two loads.
__device__ __forceinline__ int oob_unless(bool ok, int off) {
  const int mask = ok ? 0 : kOOB;
  int r;
  asm volatile("v_or_b32 %0, %1, %2" : "=v"(r) : "v"(off), "v"(mask));
  return r;
}

template <int FMT>
__device__ __forceinline__ float load_scale(const FwdArgs& p, int64_t e, int64_t n, int64_t k) {
  if constexpr (FMT == kNF4) {
    const float* s = static_cast<const float*>(p.S);
    return s[e * p.sse + n * p.ssn + (k >> 6)];
  } else {
    const uint8_t* s = static_cast<const uint8_t*>(p.S);
    return e8m0_to_f32(s[e * p.sse + n * p.ssn + (k >> 5)]);
  }
}

// Unit kinds of the decode body.
//   kPlain   out = a . W^T over the unit's 16 * kTiles rows.
//   kFfnGu   fused FFN, first stage: tile 0 holds 16 gate rows (n), tile 1
//            the matching up rows (H + n); the epilogue writes
//            h = bf16(silu_locked(bf16(gate)) * bf16(up)) instead of gu.
//   kFfnDn   fused FFN, second stage: a plain unit over h whose weight
//            loads are issued before it waits for h to be complete.
constexpr int kPlain = 0, kFfnGu = 1, kFfnDn = 2;
constexpr int kFfnFlagBase = 16;   // first flag word of the fused FFN's sync buffer

struct NoWait {
  __device__ void operator()(int*) const {}
};

// Decode LDS: [table (NF4: 64 KiB)][status word, 16 B][activations][zero block]
constexpr int kDecodeFlagBytes = 16;

// The locked fp32 silu of the fused FFN: a fixed op sequence, no FMA
// (this file builds with -ffp-contract=off), IEEE division. Same steps as
// the reference's gnf4_native/cpu_kernels.c:797-822 ("gnf4-silu-horner6/1").
__device__ __forceinline__ float silu_locked(float x) {
  if (x > 87.0f) return x;
  if (x < -87.0f) return 0.0f;
  const float t = x * -1.442695040888963e0f;
  const float n = floorf(t + 0.5f);
  const float f = t - n;
  float q = 1.535336188319500e-4f;
  q = q * f + 1.339887440266574e-3f;
  q = q * f + 9.618437357674640e-3f;
  q = q * f + 5.550332471162809e-2f;
  q = q * f + 2.402264791363012e-1f;
  q = q * f + 6.931472028550421e-1f;
  q = q * f + 1.0f;
  const float e = q * __uint_as_float((uint32_t)((int)n + 127) << 23);
  return x * (1.0f / (1.0f + e));
}

__device__ __forceinline__ float bf16_round(float f) {
  return __uint_as_float((uint32_t)f32_to_bf16_bits(f) << 16);
}

// ---- one-row (GEMV) summation order, shared by every kernel that computes
// an NF4 group of exactly one row (k_gemv_nf4, and decode_unit with row
// sets 0, which the fused FFN runs), so their outputs are bit-identical.
// A row of K elements is PR = K / 32 pieces of 32 elements (16 packed bytes).
//   * piece p: h_p = (d0 + d1) + (d2 + d3), where byte m (0..15) of the
//     piece adds LUT[hi] * a[2m] to chain 2 (m % 2) and LUT[lo] * a[2m + 1]
//     to chain 2 (m % 2) + 1 (fp32 FMAs, bytes in order), and x_p = h_p *
//     absmax[p / 2] (one fp32 multiply);
//   * slots: LR = 32 lanes for PR <= 32, else 64; slot j sums x_j, x_{j+LR},
//     x_{j+2LR}, ... in that order (pieces past the row add nothing, a slot
//     with no piece holds +0);
//   * the LR slots are added by a fixed tree: pairs (j, j ^ 32) (LR = 64),
//     then (j, j ^ 16), (j, j ^ 8), (j, j ^ 7) within eight, (j, j ^ 2),
//     (j, j ^ 1).
// The tree is what a wave's cross-lane reduction computes (group_sum).
__device__ __forceinline__ int onerow_slots(int K) { return (K >> 5) <= 32 ? 32 : 64; }

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over aligned groups of LR lanes in the tree order above; every lane of
// a group gets the group's sum (each pair is added in both lanes, a + b ==
// b + a).
template <int LR>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LR >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (LR >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (LR >= 16) v = v + dpp_f32<0x128>(v);   // row_ror:8, lane j ^ 8
  if constexpr (LR >= 8) v = v + dpp_f32<0x141>(v);    // row_half_mirror, lane j ^ 7
  if constexpr (LR >= 4) v = v + dpp_f32<0x4E>(v);     // quad_perm [2,3,0,1]
  if constexpr (LR >= 2) v = v + dpp_f32<0xB1>(v);     // quad_perm [1,0,3,2]
  return v;
}

// One decode unit: (group g, kTiles x 16 weight rows). The workgroup's
// kDecodeWaves waves split the unit's 128-element K chunks into contiguous
// runs (wave w takes chunks w * kChunksPerWave, ...). Every buffer load costs
// the CU's vector-memory front end about the same whatever its lane mask, so
// the body keeps their number low:
//   * with kAPieces > 0 (groups of at most two rows) the group's activation
//     rows are staged once per workgroup into LDS (a few 16-byte loads per
//     thread) in a [k / 8][row] layout and each MFMA A operand is a 16-byte
//     LDS read (rows that carry nothing read a zero block); with
//     kAPieces == 0 (larger groups) the operands are loaded straight into
//     registers with the weights;
//   * each weight load moves 16 bytes per lane (32 elements of one row);
//   * an NF4 lane's absmax values for a whole run are one 16-byte load;
// and issues all of them before the first wait.
//
// NF4 rows of the MFMA output. A lane of quarter q holds 32 elements of a
// 128-element chunk, so quarters 0-1 cover the chunk's first absmax block
// and quarters 2-3 its second. The A operand keeps the blocks apart: A row r
// carries token (r % 8) + 8 s of row set s, and only in the quarters of
// block r / 8 (zeros elsewhere). Output rows 0-7 are then the first block's
// sums and rows 8-15 the second's, which are exactly the rows the lane's
// quarter holds (rows 4 q .. 4 q + 3), so each lane multiplies its chunk sums
// by its own absmax in fp32 and accumulates them. Groups of up to 8 rows need
// one row set, groups of up to 16 two (twice the MFMAs). The three codebook
// parts (hi, mid, lo) go through three MFMAs per k-slice.
// NF4 groups of one row (kSets == 0, the GEMV of decode proper) skip the
// MFMA: each lane owns one weight row and 32 elements of one absmax block,
// looks up fp32 codebook pairs in the pair table (init_pair_table), forms
// the fp32 dot product with fp32 FMAs, and scales it by absmax once per
// block -- the reference GEMV's arithmetic with all 64 lanes doing useful
// work and no operand assembly.
// MXFP4 keeps 16 token rows per MFMA: its weights are exact in bf16 and the
// e8m0 scale is applied by the conversion instruction.
//
// The waves reduce their partial tiles through LDS in wave order
// (deterministic); for NF4 each lane's value is the sum of its block-0 and
// block-1 rows. The summation order of an output depends on K only, never on
// the unit kind or on which tile the row sits in.
//
// Dynamic LDS: [NF4 split or pair table 64 KiB][status word][activations
// M * K * 2][zero block]; the reduction buffer reuses the start once the
// table is no longer read. `lut` is the lane's codebook register
// (nf4_lut_lane). `ffn_h` is H and `ffn_epoch` the flag value of this call
// for kFfnGu. `wait_acts(status)` runs, in every thread, after the first
// round's weight loads are issued and before any activation load (kFfnDn);
// it leaves a nonzero status word if the unit's inputs never became ready,
// and the unit then writes NaN instead of its outputs.
template <int FMT, int kChunksPerWave, int kTiles, int kDecodeWaves, int kAPieces, int kKind,
          int kSets, class Wait>
__device__ __forceinline__ void decode_unit(const FwdArgs& p, const int g, const int64_t nu,
                                            char* smem, const int lut, const int64_t ffn_h,
                                            const int64_t ffn_n_dn, uint32_t* ffn_sync,
                                            const uint32_t ffn_epoch, const Wait& wait_acts) {
  // kFfnDn reads h, written by other workgroups during this launch, with
  // device-scope loads
  constexpr int kActAux = kKind == kFfnDn ? kScopeDevice : 0;
  static_assert(kKind != kFfnGu || (FMT == kNF4 && kTiles == 2), "gate/up pairs need 2 tiles");
  static_assert(kSets == 1 || (FMT == kNF4 && kSets == 2 && kAPieces == 0) ||
                    (FMT == kNF4 && kSets == 0 && kAPieces > 0),
                "row sets");
  constexpr bool kOneRow = kSets == 0;
  constexpr bool kSplit = FMT == kNF4 && !kOneRow;
  constexpr int kSetsA = kSets > 0 ? kSets : 1;     // activation operand sets
  constexpr int kThreadsD = 64 * kDecodeWaves;
  constexpr bool kLateActs = kKind == kFfnDn;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int q = lane >> 4;
  // split table base (LDS address 0 here: bits 8..15 free for the byte) |
  // lane column; one v_perm_b32 inserts the byte
  // (pair table: 32 columns of 8 bytes)
  const unsigned lane_off =
      (unsigned)(uintptr_t)smem |
      (kOneRow ? (unsigned)(lane & 31) * 8u : (unsigned)(lane & (kSplitCols - 1)) * 16u);
  constexpr int kScaleBytes = FMT == kNF4 ? 4 : 1;
  // NF4: A row nl carries token (nl & 7) (+ 8 per row set) in the quarters of
  // block nl / 8 only
  const bool blk_lane = !kSplit || ((nl < 8) == (q < 2));
  const int tok = kSplit ? (nl & 7) : nl;

  // the expert id and the group's rows in one round trip of scalar loads
  // (their latency heads every weight load): a null row_off reads the id
  // twice instead of branching
  const int32_t* ce = p.eids + g;
  const int32_t* cr = p.row_off ? p.row_off + (g << p.ro_shift) : ce;
  const int32_t* cr1 = p.row_off ? cr + 1 : ce;
  const int one = p.row_off ? 1 : 0;
  int e32, ro_a, ro_b;
  // (written out: the compiler otherwise waits for the id before it sends
  // the row-offset loads)
  asm volatile(
      "s_load_dword %0, %3, 0x0\n\t"
      "s_load_dword %1, %4, 0x0\n\t"
      "s_load_dword %2, %5, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(e32), "=&s"(ro_a), "=&s"(ro_b)
      : "s"(ce), "s"(cr), "s"(cr1)
      : "memory");
  const int64_t e = e32;
  const int r0 = one ? ro_a : g;
  const int M = one ? ro_b - ro_a : 1;
  if (M <= 0) return;  // uniform across the workgroup (empty group)
  const int K32 = (int)p.K;
  const int kslices = K32 >> 3;                       // 16-byte activation pieces per row
  int* const s_status = reinterpret_cast<int*>(smem + (FMT == kNF4 ? kSplitTabBytes : 0));
  const int a_base = (FMT == kNF4 ? kSplitTabBytes : 0) + kDecodeFlagBytes;
  // staged piece (k / 8, row m) at ((k / 8) M + m + k / 32) x 16 bytes: the
  // extra 16 bytes per 32 elements put the four quarters of a wave's operand
  // reads on different banks. One row: the row widened to fp32 once here
  // (32 bytes per piece, at (2 (k / 8) + k / 32) x 16), so the FMAs take
  // their operands straight from LDS.
  const int zero_off = a_base + ((kOneRow ? 2 : M) * kslices + (kslices >> 2) + 1) * 16;

  // ---- activation staging loads (first in the queue: they are waited on first)
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + (int64_t)r0 * p.lda, (int64_t)M * p.lda * 2);
  const int pieces = M * kslices;
  u32x4_t av[kAPieces > 0 ? kAPieces : 1];
  auto stage_loads = [&]() {
#pragma unroll
    for (int i = 0; i < kAPieces; ++i) {
      const int pc = (int)threadIdx.x + i * kThreadsD;
      if (wave * 64 + i * kThreadsD < pieces) {         // uniform: whole waves skip
        const int m = pc / kslices, sl = pc - m * kslices;
        av[i] = buf_load16_aux<kActAux>(
            ra, oob_unless(pc < pieces, (int)((int64_t)m * p.lda * 2) + sl * 16));
      }
    }
  };
  if constexpr (!kLateActs) stage_loads();

  // ---- weight and scale loads
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + e * p.sbe, p.N * p.sbn);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(
      static_cast<const char*>(p.S) + e * p.sse * kScaleBytes, p.N * p.ssn * kScaleBytes);
  int b_row[kTiles], s_row[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    const int64_t n = kKind == kFfnGu ? t * ffn_h + nu * 16 + nl : (nu * kTiles + t) * 16 + nl;
    b_row[t] = n < p.N ? (int)(n * p.sbn) : kOOB;
    s_row[t] = n < p.N ? (int)(n * p.ssn * kScaleBytes) : kOOB;
  }
  const int nchunks = (K32 + 127) >> 7;

  // MXFP4: two accumulators per tile (alternate k-slices). NF4: one fp32
  // accumulator per tile and row set, fed with absmax-scaled chunk sums.
  // One row: acc[t][0][0] is the lane's (row, quarter) partial.
  constexpr int kAcc = kSplit ? kSets : kOneRow ? 1 : 2;
  f32x4_t acc[kTiles][kAcc];
#pragma unroll
  for (int t = 0; t < kTiles; ++t)
#pragma unroll
    for (int s = 0; s < kAcc; ++s) acc[t][s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // one row: the lane's one-row slot sums, slot 4 (wave kChunksPerWave + i)
  // + q for the i-th chunk of each round (a round covers 32 kChunksPerWave
  // pieces, the slot count of this K: the launch picks kChunksPerWave so)
  float srow[kOneRow ? kTiles : 1][kChunksPerWave];

  // One round: this wave's chunks c0 .. c0 + kChunksPerWave - 1. All loads
  // first; in the first round the LDS staging (table, activations) happens
  // while they are in flight.
  static_assert(FMT != kNF4 || kChunksPerWave <= 2, "one 16-byte absmax load per run");
  auto round = [&](int c0, auto first_tag) {
    constexpr bool first = decltype(first_tag)::value;
    constexpr bool late = kLateActs && first;  // activations after the wait
    u32x4_t wb[kChunksPerWave][kTiles];
    unsigned sb[kChunksPerWave][kTiles];
    u32x4_t sv[kTiles];
    u32x4_t ab[kAPieces == 0 ? kChunksPerWave : 1][kSetsA][4];
    if constexpr (FMT == kNF4) {
      // absmax blocks 2 * c0 .. 2 * c0 + 3 of the lane's row: chunk c0 + i,
      // quarter q uses block 2 * (c0 + i) + q / 2
      const bool sval = (unsigned)(c0 * 128) < (unsigned)K32;
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        const int soff = oob_unless(sval, s_row[t] + c0 * 8);
        sv[t] = buf_load16(rs, soff);
      }
    }
    auto act_loads = [&](int i) {
      if constexpr (kAPieces == 0) {
        const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
        const bool kval = kseg < (unsigned)K32 && blk_lane;
#pragma unroll
        for (int s = 0; s < kSets; ++s) {
          // rows >= M fall outside the activation resource and load as zeros
          const int aoff = oob_unless(
              kval, (int)((int64_t)(tok + 8 * s) * p.lda * 2) + (int)kseg * 2);
#pragma unroll
          for (int j = 0; j < 4; ++j) ab[i][s][j] = buf_load16_aux<kActAux>(ra, aoff + 16 * j);
        }
      }
    };
#pragma unroll
    for (int i = 0; i < kChunksPerWave; ++i) {
      const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
      const bool kval = kseg < (unsigned)K32;   // also false past the last chunk
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        wb[i][t] = buf_load16(rb, oob_unless(kval, b_row[t] + (int)(kseg >> 1)));
        if constexpr (FMT != kNF4)
          sb[i][t] = buf_load1(rs, oob_unless(kval, s_row[t] + (int)(kseg >> 5)));
      }
      if constexpr (!late) act_loads(i);
    }
    if constexpr (late) {
      wait_acts(s_status);
      stage_loads();
#pragma unroll
      for (int i = 0; i < kChunksPerWave; ++i) act_loads(i);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the load block ahead of all use
    if constexpr (FMT == kNF4) {
#pragma unroll
      for (int i = 0; i < kChunksPerWave; ++i)
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
          const int idx = 2 * i + (q >> 1);   // 0..3
          sb[i][t] = idx == 0 ? sv[t][0] : idx == 1 ? sv[t][1] : idx == 2 ? sv[t][2] : sv[t][3];
        }
    }
    if constexpr (first) {
      if constexpr (kSplit) init_split_table(smem, lut);
      if constexpr (kOneRow) init_pair_table(reinterpret_cast<float2*>(smem), lut);
      if (kAPieces > 0 && threadIdx.x < 4)
        *reinterpret_cast<u32x4_t*>(smem + zero_off + threadIdx.x * 16) = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < kAPieces; ++i) {
        const int pc = (int)threadIdx.x + i * kThreadsD;
        if (wave * 64 + i * kThreadsD < pieces && pc < pieces) {
          const int m = pc / kslices, sl = pc - m * kslices;
          if constexpr (kOneRow) {
            const u32x4_t v = av[i];
            char* dst = smem + a_base + (2 * sl + (sl >> 2)) * 16;
            *reinterpret_cast<u32x4_t*>(dst) =
                u32x4_t{v[0] << 16, v[0] & 0xFFFF0000u, v[1] << 16, v[1] & 0xFFFF0000u};
            *reinterpret_cast<u32x4_t*>(dst + 16) =
                u32x4_t{v[2] << 16, v[2] & 0xFFFF0000u, v[3] << 16, v[3] & 0xFFFF0000u};
          } else {
            *reinterpret_cast<u32x4_t*>(smem + a_base + (sl * M + m + (sl >> 2)) * 16) = av[i];
          }
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kChunksPerWave; ++i) {
      const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
      const bool kval = kseg < (unsigned)K32;
      u32x4_t a[kSetsA][4];
      f32x4_t af[kOneRow ? 4 : 1][2];   // one row: fp32 activations
      if constexpr (kOneRow) {
        // every lane: the group's one row over its 32 elements
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int sl = (int)(kseg >> 3) + j;
          const int off = kval ? a_base + (2 * sl + (sl >> 2)) * 16 : zero_off;
          af[j][0] = *reinterpret_cast<const f32x4_t*>(smem + off);
          af[j][1] = *reinterpret_cast<const f32x4_t*>(smem + off + 16);
        }
      } else if constexpr (kAPieces > 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int sl = (int)(kseg >> 3) + j;
          const int off = (kval && blk_lane && tok < M)
                              ? a_base + (sl * M + tok + (sl >> 2)) * 16
                              : zero_off;
          a[0][j] = *reinterpret_cast<const u32x4_t*>(smem + off);
        }
      } else {
#pragma unroll
        for (int s = 0; s < kSets; ++s)
#pragma unroll
          for (int j = 0; j < 4; ++j) a[s][j] = ab[i][s][j];
      }
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        if constexpr (kOneRow) {
          // fp32 codebook pairs times fp32 activations, four chains
          float d[4] = {0.f, 0.f, 0.f, 0.f};
          // all 16 lookups in flight before the first FMA
          f32x2_t w[16];
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b)
              w[4 * j + b] = lds_read8f(
                  __builtin_amdgcn_perm(wb[i][t][j], lane_off, 0x0C0C0000u | ((4u + b) << 8)));
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              const f32x4_t& x = af[j][b >> 1];
              d[2 * (b & 1)] = __builtin_fmaf(w[4 * j + b][0], x[2 * (b & 1)], d[2 * (b & 1)]);
              d[2 * (b & 1) + 1] =
                  __builtin_fmaf(w[4 * j + b][1], x[2 * (b & 1) + 1], d[2 * (b & 1) + 1]);
            }
          const float xv = ((d[0] + d[1]) + (d[2] + d[3])) * __uint_as_float(sb[i][t]);
          if constexpr (first) srow[t][i] = kval ? xv : 0.0f;
          else srow[t][i] = kval ? srow[t][i] + xv : srow[t][i];
        } else if constexpr (kSplit) {
          // chunk sums of the three parts, two chains per row set
          f32x4_t c[kSets][2];
#pragma unroll
          for (int s = 0; s < kSets; ++s) c[s][0] = c[s][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            u32x4_t hi, mid, lo;
            split_lookup(wb[i][t][j], lane_off, hi, mid, lo);
#pragma unroll
            for (int s = 0; s < kSets; ++s) {
              c[s][j & 1] = mfma(a[s][j], hi, c[s][j & 1]);
              c[s][j & 1] = mfma(a[s][j], mid, c[s][j & 1]);
              c[s][j & 1] = mfma(a[s][j], lo, c[s][j & 1]);
            }
          }
          const float am = __uint_as_float(sb[i][t]);
#pragma unroll
          for (int s = 0; s < kSets; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[t][s][r] = __builtin_fmaf(c[s][0][r] + c[s][1][r], am, acc[t][s][r]);
        } else {
          u32x4_t b[4];
          const float sc = e8m0_to_f32(sb[i][t]);
#pragma unroll
          for (int j = 0; j < 4; ++j) b[j] = mx_dword_to_bf16(wb[i][t][j], sc);
          acc[t][0] = mfma(a[0][0], b[0], acc[t][0]);
          acc[t][1] = mfma(a[0][1], b[1], acc[t][1]);
          acc[t][0] = mfma(a[0][2], b[2], acc[t][0]);
          acc[t][1] = mfma(a[0][3], b[3], acc[t][1]);
        }
      }
    }
  };
  // every wave runs the first round: chunks past the end load zeros
  round(wave * kChunksPerWave, std::true_type{});
  for (int c0 = (kDecodeWaves + wave) * kChunksPerWave; c0 < nchunks;
       c0 += kDecodeWaves * kChunksPerWave)
    round(c0, std::false_type{});

  __syncthreads();  // the table is no longer read: its space takes the partials
  f32x4_t* s_red = reinterpret_cast<f32x4_t*>(smem);   // [kDecodeWaves][kTiles][kSetsA][64]
  // one row: slots [kTiles * 16][kSlots + 1], then the row sums
  constexpr int kSlots = 32 * kChunksPerWave;
  float* s_slot = reinterpret_cast<float*>(smem);
  float* s_tot = s_slot + kTiles * 16 * (kSlots + 1);
  static_assert(!kOneRow || kDecodeWaves == 8, "one-row slots assume eight waves");
#pragma unroll
  for (int t = 0; t < kTiles; ++t) {
    if constexpr (kOneRow) {
#pragma unroll
      for (int i = 0; i < kChunksPerWave; ++i)
        s_slot[(t * 16 + nl) * (kSlots + 1) + 4 * (wave * kChunksPerWave + i) + q] = srow[t][i];
    } else {
#pragma unroll
      for (int s = 0; s < kSetsA; ++s) {
        if constexpr (kSplit)
          s_red[((wave * kTiles + t) * kSetsA + s) * 64 + lane] = acc[t][s];
        else
          s_red[((wave * kTiles + t) * kSetsA + s) * 64 + lane] = acc[t][0] + acc[t][kAcc - 1];
      }
    }
  }
  __syncthreads();
  if constexpr (kOneRow) {
    // each row's slots through the one-row tree (64 / kSlots rows per pass)
    constexpr int kRows = kTiles * 16, kPerPass = 64 / kSlots;
    for (int r0w = wave * kPerPass; r0w < kRows; r0w += kDecodeWaves * kPerPass) {
      const int r = r0w + lane / kSlots;
      const float v = group_sum<kSlots>(s_slot[r * (kSlots + 1) + (lane % kSlots)]);
      if (lane % kSlots == 0) s_tot[r] = v;
    }
    __syncthreads();
  }
  // tile t, row set s of the output, summed over the waves in wave order;
  // NF4 lanes 0..31 add the second block's rows (lane + 32) to the first's;
  // one row: lanes 0..15 read their row's sum
  auto reduced = [&](int t, int s) {
    if constexpr (kOneRow) {
      return f32x4_t{s_tot[t * 16 + nl], 0.f, 0.f, 0.f};
    } else {
      const f32x4_t* r = s_red + (t * kSetsA + s) * 64 + lane;
      constexpr int kStride = kTiles * kSetsA * 64;
      f32x4_t v = kSplit ? r[0] + r[32] : r[0];
#pragma unroll
      for (int w = 1; w < kDecodeWaves; ++w)
        v = v + (kSplit ? r[w * kStride] + r[w * kStride + 32] : r[w * kStride]);
      return v;
    }
  };
  // output rows of lane (nl, q), i = 0..3: 8 s + 4 q + i (NF4, q < 2), 4 q + i
  // (MXFP4), or row 0 of lanes 0..15 (one row)
  const bool writer = kOneRow ? lane < 16 : (!kSplit || q < 2);
  constexpr int kRowsPerLane = kOneRow ? 1 : 4;
  if constexpr (kKind == kFfnGu) {
    // wave 0 sums the gate and up tiles over the waves in wave order and
    // writes h for its 16 columns: the same bits as a plain gu launch
    // (bf16 out) followed by the silu-multiply kernel
    if (wave == 0) {
      // h goes out with device-scope stores; once the wave's stores have
      // completed (vmcnt 0) they are visible to device-scope loads on every
      // XCD
      const __amdgpu_buffer_rsrc_t rh =
          make_rsrc(p.out + (int64_t)r0 * p.ldo, (int64_t)M * p.ldo * 2);
      const int col = (int)(nu * 16 + nl);
#pragma unroll
      for (int s = 0; s < kSetsA; ++s) {
        const f32x4_t vg = reduced(0, s), vu = reduced(1, s);
        if (writer) {
#pragma unroll
          for (int i = 0; i < kRowsPerLane; ++i) {
            const int m = 8 * s + 4 * q + i;
            const float hv = silu_locked(bf16_round(vg[i])) * bf16_round(vu[i]);
            const int off = oob_unless(m < M, (int)(((int64_t)m * p.ldo + col) * 2));
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(hv), rh, off, 0,
                                                  kScopeDevice);
          }
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      // one flag in the private row of every down unit of the group:
      // flags[(g * dn_per_group + d) * gu_per_group + nu]
      const int64_t gu_per_group = ffn_h / 16;
      const int64_t dn_per_group = (ffn_n_dn + 31) / 32;
      uint32_t* row0 = ffn_sync + kFfnFlagBase + (int64_t)g * dn_per_group * gu_per_group + nu;
      for (int64_t d = lane; d < dn_per_group; d += 64)
        __hip_atomic_store(row0 + d * gu_per_group, ffn_epoch, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    // a down unit whose h never became ready writes NaN (the status word was
    // set before the barrier that ended its wait)
    const bool poisoned = kLateActs && *s_status != 0;
    // wave t * kSetsA + s sums tile t, row set s over the waves
    if (wave < kTiles * kSetsA) {
      const int t = wave / kSetsA, s = wave - t * kSetsA;
      const int64_t n = (nu * kTiles + t) * 16 + nl;
      const f32x4_t v = reduced(t, s);
      if (writer && n < p.N) {
#pragma unroll
        for (int i = 0; i < kRowsPerLane; ++i) {
          const int m = (kSplit ? 8 * s : 0) + 4 * q + i;
          if (m < M)
            p.out[(int64_t)(r0 + m) * p.ldo + n] = poisoned ? (uint16_t)0x7FC0 : f32_to_bf16_bits(v[i]);
        }
      }
    }
  }
}

// Decode path: one unit per workgroup.
template <int FMT, int kChunksPerWave, int kTiles, int kDecodeWaves, int kAPieces, int kSets>
// two workgroups per CU: kDecodeWaves / 2 waves per SIMD
// The grid is (units per group, G): the unit is read off the block
// coordinates, with no division (G <= 65535 on this path).
__global__ void __launch_bounds__(64 * kDecodeWaves, kDecodeWaves / 2) k_decode_fwd(const FwdArgs p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int lut = FMT == kNF4 ? nf4_lut_lane() : 0;
  __builtin_amdgcn_sched_barrier(0);  // the codebook load goes out first
  // every argument the unit needs, fetched in one round trip before the
  // expert id (left to itself the compiler fetches them in several rounds,
  // each behind a branch)
  const FwdArgs q = p;
  asm volatile("" ::"s"(q.a), "s"(q.lda), "s"(q.B), "s"(q.sbe), "s"(q.sbn), "s"(q.S), "s"(q.sse),
               "s"(q.ssn), "s"(q.eids), "s"(q.row_off), "s"(q.ro_shift), "s"(q.N), "s"(q.K), "s"(q.out),
               "s"(q.ldo));
  const int g = (int)blockIdx.y;   // < G: the grid has exactly G rows of units
  decode_unit<FMT, kChunksPerWave, kTiles, kDecodeWaves, kAPieces, kPlain, kSets>(
      q, g, (int64_t)blockIdx.x, smem, lut, 0, 0, nullptr, 0u, NoWait{});
}

// A workgroup barrier for LDS only: waits for this wave's LDS operations
// (lgkmcnt 0), not for its global loads in flight -- __syncthreads() also
// fences global memory, which waits for every outstanding load. The empty
// asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ------------------------------------------------------ one-row GEMV --
//
// k_gemv_nf4<LR, PPL, RPW>: NF4 decode where every group is one row (the
// reference's GEMV, kernel/nf4_grouped.py:465-514), in the one-row
// summation order above. Lanes run along the weight row: a lane owns
// pieces j, j + LR, ... (j = lane % LR, PPL of them) of one row, so a wave
// load of 16 bytes per lane reads 64 / LR rows of LR x 16 contiguous bytes
// (whole cache lines), and the lane's activations (32 PPL of them) are
// loaded once, widened to fp32 and kept in registers for every row it
// visits. Each wave walks RPW row steps of 64 / LR rows; a workgroup of
// eight waves covers 8 RPW (64 / LR) rows of one group (grid: row blocks x
// groups).
//   * The wave keeps two row steps of loads in flight and issues step s + 2
//     before it decodes step s. Vector-memory instructions issue in order,
//     so when the memory system pushes back the wave stalls at its next
//     load: the codebook table is therefore built after the first two
//     steps' loads, not after all of them, and its barrier comes early.
//   * The pair table (as init_pair_table, 32 lane columns) is filled from
//     immediate codebook constants: no memory load precedes it.
//   * A row's slots are added across the LR lanes with group_sum; lane
//     j == s of each row group keeps step s's sum, so one store per wave
//     writes its rows' contiguous outputs.
// Bound: HBM bytes plus one LDS lookup per packed byte (35 lane lookups
// per ns per CU measured on MI355X). Algorithmic bytes per workgroup:
// rows x (K / 2 + K / 16).
// GU: the expert FFN's first stage for one-row groups: gate row n and up row
// H + n (ffn_h = H) on consecutive steps 2 i, 2 i + 1 of one wave, and the
// epilogue writes h[n] = bf16(silu_locked(bf16(gate)) * bf16(up)) to `out`
// (ldo) instead of the gate_up row: the bits of a plain launch followed by
// k_silu_mul. RPW is even there; a wave covers RPW / 2 columns of h per row
// group.
// ROWS: groups of up to four rows, one row per pass (a later pass reads the
// same weight rows again, from L2, and decodes them again): each row's sums
// follow the one-row order, so a row's bits do not depend on its group's
// size. (Passes of two and four rows, with the activations held packed or
// widened, were slower on MI355X: their registers halve the waves per SIMD,
// and the lost latency hiding costs more than the repeated decode.)
template <int LR, int PPL, int RPW, bool GU = false, bool ROWS = false>
__global__ void __launch_bounds__(512, PPL >= 3 ? 1 : 2) k_gemv_nf4(const FwdArgs p,
                                                                    const int ffn_h,
                                                                    const GemvIds gi) {
  static_assert(!GU || RPW % 2 == 0, "gate / up step pairs");
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int RS = 64 / LR;          // rows per wave step
  constexpr int D = RPW < 2 ? RPW : 2; // row steps in flight
  const FwdArgs q = p;
  // kernel-argument ids: loaded with the other arguments, in one round trip
  // (a clamped index keeps every load inside the arguments)
  const int gc = (int)blockIdx.y < kGemvIdsMax ? (int)blockIdx.y : kGemvIdsMax - 1;
  const int gi_n = gi.n, gi_e = gi.e[gc], gi_rows = gi.rows[gc];
  asm volatile("" ::"s"(q.a), "s"(q.lda), "s"(q.B), "s"(q.sbe), "s"(q.sbn), "s"(q.S), "s"(q.sse),
               "s"(q.ssn), "s"(q.eids), "s"(q.row_off), "s"(q.ro_shift), "s"(q.N), "s"(q.K), "s"(q.out),
               "s"(q.ldo), "s"(gi_n), "s"(gi_e), "s"(gi_rows));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rl = lane / LR, j = lane % LR;
  const int g = (int)blockIdx.y;
  // the expert id and the group's row in one round trip of scalar loads
  int e32, ro_a, ro_b;
  bool has_ro;
  if (gi_n > 0) {   // ids in the kernel arguments
    has_ro = true;
    e32 = gi_e;
    ro_a = gi_rows >> 8;
    ro_b = ro_a + (gi_rows & 0xFF);
  } else {
    has_ro = q.row_off != nullptr;
    const int32_t* ce = q.eids + g;
    const int32_t* cr = has_ro ? q.row_off + (g << q.ro_shift) : ce;
    const int32_t* cr1 = has_ro ? cr + 1 : ce;
    asm volatile(
        "s_load_dword %0, %3, 0x0\n\t"
        "s_load_dword %1, %4, 0x0\n\t"
        "s_load_dword %2, %5, 0x0\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(e32), "=&s"(ro_a), "=&s"(ro_b)
        : "s"(ce), "s"(cr), "s"(cr1)
        : "memory");
  }
  const int r0 = has_ro ? ro_a : g;
  if (has_ro && ro_b - ro_a <= 0) return;   // empty group (uniform)
  const int64_t e = e32;
  const int K32 = (int)q.K;
  const int PR = K32 >> 5;
  const int N32 = (int)q.N;
  // (GU: wrow0 counts columns of h, RPW / 2 per wave and row slot)
  constexpr int kCols = GU ? RPW / 2 : RPW;
  const int wrow0 = (int)blockIdx.x * (8 * kCols * RS) + wave * (kCols * RS);
  // weight row of step s, and whether it is inside the matrix
  auto step_row = [&](int s) {
    return GU ? (s & 1) * ffn_h + wrow0 + (s >> 1) * RS + rl : wrow0 + s * RS + rl;
  };
  auto step_ok = [&](int s) {
    return GU ? wrow0 + (s >> 1) * RS + rl < ffn_h : wrow0 + s * RS + rl < N32;
  };
  // one pass over the workgroup's weight rows for group row rm (build: the
  // first pass, which builds the table)
  auto pass = [&](const int rm, const bool build) {
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(q.a + (int64_t)rm * q.lda, (int64_t)K32 * 2);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(q.B + e * q.sbe, q.N * q.sbn);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(static_cast<const char*>(q.S) + e * q.sse * 4,
                                                q.N * q.ssn * 4);
    // activations of the lane's pieces (64 bytes each), first in the queue
    u32x4_t av[PPL][4];
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int pc = j + i * LR;
#pragma unroll
      for (int t = 0; t < 4; ++t) av[i][t] = buf_load16(ra, oob_unless(pc < PR, pc * 64 + t * 16));
    }
    u32x4_t wb[RPW][PPL];
    unsigned sa[RPW][PPL];
    auto issue = [&](int s) {
      const int n = step_row(s);
      const bool row_ok = step_ok(s);
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        const int pc = j + i * LR;
        const bool ok = row_ok && pc < PR;
        wb[s][i] = buf_load16(rb, oob_unless(ok, n * (int)q.sbn + pc * 16));
        sa[s][i] = __builtin_amdgcn_raw_buffer_load_b32(
            rs, oob_unless(ok, (n * (int)q.ssn + (pc >> 1)) * 4), 0, 0);
      }
    };
#pragma unroll
    for (int s = 0; s < D; ++s) issue(s);
    __builtin_amdgcn_sched_barrier(0);
    if (build) {   // uniform: the table once per workgroup
      init_pair_table_imm(smem);
      lds_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    // widen the activations once
    f32x4_t af[PPL][8];
#pragma unroll
    for (int i = 0; i < PPL; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const u32x4_t x = av[i][t];
        af[i][2 * t] = f32x4_t{__uint_as_float(x[0] << 16), __uint_as_float(x[0] & 0xFFFF0000u),
                               __uint_as_float(x[1] << 16), __uint_as_float(x[1] & 0xFFFF0000u)};
        af[i][2 * t + 1] = f32x4_t{__uint_as_float(x[2] << 16), __uint_as_float(x[2] & 0xFFFF0000u),
                                   __uint_as_float(x[3] << 16), __uint_as_float(x[3] & 0xFFFF0000u)};
      }
    const unsigned lane_off = (unsigned)(uintptr_t)smem | (unsigned)(lane & 31) * 8u;
    float v[RPW];
#pragma unroll
    for (int s = 0; s < RPW; ++s) {
      if (s + D < RPW) issue(s + D);
      __builtin_amdgcn_sched_barrier(0);
      float slot = 0.0f;
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        f32x2_t w[16];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b)
            w[4 * jj + b] = lds_read8f(
                __builtin_amdgcn_perm(wb[s][i][jj], lane_off, 0x0C0C0000u | ((4u + b) << 8)));
        float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const f32x4_t& x = af[i][2 * jj + (b >> 1)];
            d[2 * (b & 1)] = __builtin_fmaf(w[4 * jj + b][0], x[2 * (b & 1)], d[2 * (b & 1)]);
            d[2 * (b & 1) + 1] =
                __builtin_fmaf(w[4 * jj + b][1], x[2 * (b & 1) + 1], d[2 * (b & 1) + 1]);
          }
        const float xv = ((d[0] + d[1]) + (d[2] + d[3])) * __uint_as_float(sa[s][i]);
        const bool valid = j + i * LR < PR;
        if (i == 0) slot = valid ? xv : 0.0f;
        else slot = valid ? slot + xv : slot;
      }
      v[s] = group_sum<LR>(slot);
    }
    if constexpr (GU) {
      float ov = 0.0f;
#pragma unroll
      for (int c = 0; c < kCols; ++c) {
        const float hv = silu_locked(bf16_round(v[2 * c])) * bf16_round(v[2 * c + 1]);
        ov = j == c ? hv : ov;
      }
      const int n = wrow0 + j * RS + rl;
      if (j < kCols && n < ffn_h) q.out[(int64_t)rm * q.ldo + n] = f32_to_bf16_bits(ov);
    } else {
      float ov = v[0];
#pragma unroll
      for (int s = 1; s < RPW; ++s) ov = j == s ? v[s] : ov;
      const int n = wrow0 + j * RS + rl;
      if (j < RPW && n < N32) q.out[(int64_t)rm * q.ldo + n] = f32_to_bf16_bits(ov);
    }
  };
  if constexpr (!ROWS) {
    pass(r0, true);
  } else {
    // every row of the group in turn (one row without row offsets)
    const int m_all = has_ro ? ro_b - ro_a : 1;
    for (int m = 0; m < m_all; ++m) pass(r0 + m, m == 0);
  }
}

// k_gemv_mx<LR, PPL, RPW>: the same row-major walk for MXFP4 groups of one
// row (reference kernel/mxfp4_grouped.py:100-131). A 16-byte piece is one
// e8m0 scale block; v_cvt_scalef32_pk_bf16_fp4 turns each packed byte into
// a bf16 pair already scaled by 2^(e - 127) (exact), and v_dot2_f32_bf16
// multiplies it with the activation pair and adds it into one of four fp32
// chains. No table, so no LDS and no barrier: the wave issues its first two
// row steps and starts on the first as soon as it lands.
// One-row MXFP4 order: piece p: h_p = (d0 + d1) + (d2 + d3), chain c taking
// the dot of byte 4 j + c for j = 0..3 in order; slots and tree as the NF4
// one-row order, with LR chosen per K by the launch (mx_slots).
// (The activation pairs are taken out of a bf16x8 view of each 16-byte
// chunk by element shuffles: hipcc 7.2 folds a bit_cast of dword 1..3 of a
// u32x4 into a bf16x2 to dword 0.)
template <int LR, int PPL, int RPW>
__global__ void __launch_bounds__(512, 2) k_gemv_mx(const FwdArgs p, const GemvIds gi) {
  constexpr int RS = 64 / LR;
  constexpr int D = RPW < 2 ? RPW : 2;
  const FwdArgs q = p;
  // kernel-argument ids: loaded with the other arguments, in one round trip
  // (a clamped index keeps every load inside the arguments)
  const int gc = (int)blockIdx.y < kGemvIdsMax ? (int)blockIdx.y : kGemvIdsMax - 1;
  const int gi_n = gi.n, gi_e = gi.e[gc], gi_rows = gi.rows[gc];
  asm volatile("" ::"s"(q.a), "s"(q.lda), "s"(q.B), "s"(q.sbe), "s"(q.sbn), "s"(q.S), "s"(q.sse),
               "s"(q.ssn), "s"(q.eids), "s"(q.row_off), "s"(q.ro_shift), "s"(q.N), "s"(q.K), "s"(q.out),
               "s"(q.ldo), "s"(gi_n), "s"(gi_e), "s"(gi_rows));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rl = lane / LR, j = lane % LR;
  const int g = (int)blockIdx.y;
  int e32, ro_a, ro_b;
  bool has_ro;
  if (gi_n > 0) {   // ids in the kernel arguments
    has_ro = true;
    e32 = gi_e;
    ro_a = gi_rows >> 8;
    ro_b = ro_a + (gi_rows & 0xFF);
  } else {
    has_ro = q.row_off != nullptr;
    const int32_t* ce = q.eids + g;
    const int32_t* cr = has_ro ? q.row_off + (g << q.ro_shift) : ce;
    const int32_t* cr1 = has_ro ? cr + 1 : ce;
    asm volatile(
        "s_load_dword %0, %3, 0x0\n\t"
        "s_load_dword %1, %4, 0x0\n\t"
        "s_load_dword %2, %5, 0x0\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(e32), "=&s"(ro_a), "=&s"(ro_b)
        : "s"(ce), "s"(cr), "s"(cr1)
        : "memory");
  }
  const int r0 = has_ro ? ro_a : g;
  if (has_ro && ro_b - ro_a <= 0) return;   // empty group (uniform)
  const int64_t e = e32;
  const int K32 = (int)q.K;
  const int PR = K32 >> 5;
  const int N32 = (int)q.N;
  const int wrow0 = (int)blockIdx.x * (8 * RPW * RS) + wave * (RPW * RS);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(q.a + (int64_t)r0 * q.lda, (int64_t)K32 * 2);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(q.B + e * q.sbe, q.N * q.sbn);
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(static_cast<const uint8_t*>(q.S) + e * q.sse, q.N * q.ssn);
  u32x4_t av[PPL][4];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int pc = j + i * LR;
#pragma unroll
    for (int t = 0; t < 4; ++t) av[i][t] = buf_load16(ra, oob_unless(pc < PR, pc * 64 + t * 16));
  }
  u32x4_t wb[RPW][PPL];
  unsigned sb[RPW][PPL];
  auto issue = [&](int s) {
    const int n = wrow0 + s * RS + rl;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int pc = j + i * LR;
      const bool ok = n < N32 && pc < PR;
      wb[s][i] = buf_load16(rb, oob_unless(ok, n * (int)q.sbn + pc * 16));
      sb[s][i] = buf_load1(rs, oob_unless(ok, n * (int)q.ssn + pc));
    }
  };
#pragma unroll
  for (int s = 0; s < D; ++s) issue(s);
  float v[RPW];
#pragma unroll
  for (int s = 0; s < RPW; ++s) {
    if (s + D < RPW) issue(s + D);
    __builtin_amdgcn_sched_barrier(0);
    float slot = 0.0f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const float sc = e8m0_to_f32(sb[s][i]);
      float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const unsigned x = wb[s][i][jj];
        const bf16x8_t a8 = as_bf16x8(av[i][jj]);
        d[0] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 0),
                                               __builtin_shufflevector(a8, a8, 0, 1), d[0], false);
        d[1] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 1),
                                               __builtin_shufflevector(a8, a8, 2, 3), d[1], false);
        d[2] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 2),
                                               __builtin_shufflevector(a8, a8, 4, 5), d[2], false);
        d[3] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 3),
                                               __builtin_shufflevector(a8, a8, 6, 7), d[3], false);
      }
      const float xv = (d[0] + d[1]) + (d[2] + d[3]);
      const bool valid = j + i * LR < PR;
      if (i == 0) slot = valid ? xv : 0.0f;
      else slot = valid ? slot + xv : slot;
    }
    v[s] = group_sum<LR>(slot);
  }
  float ov = v[0];
#pragma unroll
  for (int s = 1; s < RPW; ++s) ov = j == s ? v[s] : ov;
  const int n = wrow0 + j * RS + rl;
  if (j < RPW && n < N32) q.out[(int64_t)r0 * q.ldo + n] = f32_to_bf16_bits(ov);
}

// ------------------------------------------------- row-streaming decode --
//
// k_decode_rows<FMT, kW, kT, kSets, kCpw, kR, kP, kAbsBlock>: decode (every group <= 16
// rows) for launches with many groups (batched decode). Each wave owns
// 16 kT weight rows of one group over the whole K, so no partial sums cross
// waves: the wave streams its rows' 128-element chunks through a register
// ring of kD = kCpw * kR chunks of loads in flight (16 bytes of packed
// weights per lane and tile; NF4 absmax once per chunk pair, 16 bytes),
// decodes and multiplies each chunk as it lands, and refills the slot with
// the chunk kD ahead. The ring loop is straight-line code (chunks past the
// end load zeros and add nothing), so the loads stay in flight across
// iterations. A workgroup of kW waves covers 16 kT kW rows of one group:
// its activation rows (at most kP 16-byte pieces per thread) are staged
// once into LDS, next to the NF4 split table, while the first chunks are in
// flight. Staged layout: piece (k / 8, row m) at ((k / 8) M + m + k / 32)
// x 16 bytes -- the extra 16 bytes per 32 elements put the four quarters of
// a wave's operand reads on different banks -- then a zero block.
// Bits: the MFMA row semantics and operands are those of decode_unit (NF4:
// rows 0-7 and 8-15 hold the two absmax blocks of a chunk for tokens
// 8 s + 0..7; MXFP4: 16 token rows), and the wave folds its chunk sums in
// decode_unit's order: chunks in runs of kCpw (the run wave w of a
// k_decode_fwd launch takes when the launch needs one round), each run
// summed in its own chain, the runs added in order. So both kernels -- and
// the fused FFN, which runs decode_unit -- give identical outputs.
template <int FMT, int kW, int kT, int kSets, int kCpw, int kR, int kP, bool kAbsBlock>
__global__ void __launch_bounds__(64 * kW, 4) k_decode_rows(const FwdArgs p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr bool kSplit = FMT == kNF4;
  static_assert(kSets == 1 || (kSplit && kSets == 2), "row sets");
  constexpr int kD = kCpw * kR;
  static_assert(!kSplit || kD % 2 == 0, "NF4 absmax comes per chunk pair");
  constexpr int kScaleBytes = FMT == kNF4 ? 4 : 1;
  const int lut = FMT == kNF4 ? nf4_lut_lane() : 0;
  __builtin_amdgcn_sched_barrier(0);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int q = lane >> 4;
  const int g = (int)blockIdx.y;

  const int32_t* ce = p.eids + g;
  const int32_t* cr = p.row_off ? p.row_off + (g << p.ro_shift) : ce;
  const int32_t* cr1 = p.row_off ? cr + 1 : ce;
  const int one = p.row_off ? 1 : 0;
  int e32, ro_a, ro_b;
  asm volatile(
      "s_load_dword %0, %3, 0x0\n\t"
      "s_load_dword %1, %4, 0x0\n\t"
      "s_load_dword %2, %5, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(e32), "=&s"(ro_a), "=&s"(ro_b)
      : "s"(ce), "s"(cr), "s"(cr1)
      : "memory");
  const int64_t e = e32;
  const int r0 = one ? ro_a : g;
  const int M = one ? ro_b - ro_a : 1;
  if (M <= 0) return;  // uniform across the workgroup (empty group)
  const int K32 = (int)p.K;
  const int nchunks = (K32 + 127) >> 7;

  // ---- activation staging loads first: they are waited on first
  const int a_base = FMT == kNF4 ? kSplitTabBytes : 0;
  const int kslices = K32 >> 3;
  const int pieces = M * kslices;
  const int zero_off = a_base + (pieces + (kslices >> 2) + 1) * 16;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + (int64_t)r0 * p.lda, (int64_t)M * p.lda * 2);
  u32x4_t av[kP];
#pragma unroll
  for (int j = 0; j < kP; ++j) {
    const int pc = j * 64 * kW + (int)threadIdx.x;
    const int m = pc / kslices, sl = pc - m * kslices;
    av[j] = buf_load16(ra, oob_unless(pc < pieces, (int)((int64_t)m * p.lda * 2) + sl * 16));
  }

  // ---- the ring's first kD chunks
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + e * p.sbe, p.N * p.sbn);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(
      static_cast<const char*>(p.S) + e * p.sse * kScaleBytes, p.N * p.ssn * kScaleBytes);
  int64_t n[kT];
  int b_row[kT], s_row[kT];
#pragma unroll
  for (int t = 0; t < kT; ++t) {
    n[t] = (int64_t)blockIdx.x * (16 * kW * kT) + (wave * kT + t) * 16 + nl;
    b_row[t] = n[t] < p.N ? (int)(n[t] * p.sbn) + q * 16 : kOOB;
    // NF4: the row's absmax (blocks 4 h .. 4 h + 3 of chunk pair h); MXFP4:
    // the lane's scale byte (block 4 c + q)
    s_row[t] = n[t] < p.N ? (int)(n[t] * p.ssn * kScaleBytes) + (FMT == kNF4 ? 0 : q) : kOOB;
  }
  u32x4_t wr[kD][kT];
  u32x4_t sq[kSplit && !kAbsBlock ? kD / 2 : 1][kT];   // NF4 absmax of chunk pairs
  unsigned sb[kSplit ? 1 : kD][kT];      // MXFP4 scale bytes
  // NF4 with kAbsBlock: the absmax of a tile's 16 rows (16 x K / 64 floats,
  // contiguous, at most 1 KiB) comes in as one coalesced load, ahead of the
  // ring, lane L holding floats 4 L .. 4 L + 3; a chunk pair's four floats
  // of row nl then sit in one lane (the row length is a multiple of 4) and
  // reach lane (nl, q) through four ds_bpermute. The per-pair loads put 16
  // rows' lines into each load: as many requests as the weight loads.
  constexpr bool abs_block = kSplit && kAbsBlock;
  const int abs_row = (int)p.ssn;   // floats
  u32x4_t sgl[kT];
  if constexpr (abs_block) {
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      const int64_t n0 = (int64_t)blockIdx.x * (16 * kW * kT) + (wave * kT + t) * 16;
      sgl[t] = buf_load16(rs, oob_unless(n0 < p.N, (int)(n0 * abs_row * 4) + lane * 16));
    }
  }
  auto issue = [&](int c, int slot) {
    // past the end of K (the second half of a last 64-element chunk, or the
    // ring's refills beyond the last chunk): zeros
    const bool ok = (unsigned)(c * 128 + q * 32) < (unsigned)K32;
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      wr[slot][t] = buf_load16(rb, oob_unless(ok, b_row[t] + c * 64));
      if constexpr (kSplit) {
        if constexpr (!abs_block)
          if ((slot & 1) == 0)
          sq[slot / 2][t] = buf_load16(rs, oob_unless((unsigned)(c * 128) < (unsigned)K32,
                                                      s_row[t] + c * 8));
      } else {
        sb[slot][t] = buf_load1(rs, oob_unless(ok, s_row[t] + c * 4));
      }
    }
  };
#pragma unroll
  for (int i = 0; i < kD; ++i) issue(i, i);

  // ---- LDS: [NF4 split table][activations M x K, padded][zero block]
#pragma unroll
  for (int j = 0; j < kP; ++j) {
    const int pc = j * 64 * kW + (int)threadIdx.x;
    if (pc < pieces) {
      const int m = pc / kslices, sl = pc - m * kslices;
      *reinterpret_cast<u32x4_t*>(smem + a_base + (sl * M + m + (sl >> 2)) * 16) = av[j];
    }
  }
  if (threadIdx.x < 4)
    *reinterpret_cast<u32x4_t*>(smem + zero_off + threadIdx.x * 16) = u32x4_t{0u, 0u, 0u, 0u};
  if constexpr (FMT == kNF4) init_split_table(smem, lut);
  __syncthreads();

  // NF4: A row nl carries token (nl & 7) + 8 s in the quarters of block
  // nl / 8 only; MXFP4: token nl
  const bool blk_lane = !kSplit || ((nl < 8) == (q < 2));
  const int tok = kSplit ? (nl & 7) : nl;
  const unsigned lane_off = (unsigned)(uintptr_t)smem | (unsigned)(lane & (kSplitCols - 1)) * 16u;
  // per row set: the lane's activation row offset (or -1)
  int a_row[kSets];
#pragma unroll
  for (int s = 0; s < kSets; ++s)
    a_row[s] = (blk_lane && tok + 8 * s < M) ? a_base + (tok + 8 * s) * 16 : -1;
  // acc: the current run's chains (NF4: [t][s][0]; MXFP4: alternate
  // k-slices); tot: the runs folded so far (it starts at +0, which a first
  // run adds to exactly: no run sum is -0)
  f32x4_t acc[kT][kSets][2], tot[kT][kSets];
#pragma unroll
  for (int t = 0; t < kT; ++t)
#pragma unroll
    for (int s = 0; s < kSets; ++s)
      acc[t][s][0] = acc[t][s][1] = tot[t][s] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int c, const u32x4_t (&w)[kT], const float (&scl)[kT]) {
    const int kp = c * 16 + q * 4;   // first 16-byte activation piece of the lane's slice
    const bool kval = kp < kslices;
    u32x4_t a[kSets][4];
#pragma unroll
    for (int s = 0; s < kSets; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int off = (kval && a_row[s] >= 0)
                            ? a_row[s] + ((kp + j) * M + ((kp + j) >> 2)) * 16 : zero_off;
        a[s][j] = *reinterpret_cast<const u32x4_t*>(smem + off);
      }
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      if constexpr (kSplit) {
        f32x4_t cs[kSets][2];
#pragma unroll
        for (int s = 0; s < kSets; ++s) cs[s][0] = cs[s][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          u32x4_t hi, mid, lo;
          split_lookup(w[t][j], lane_off, hi, mid, lo);
#pragma unroll
          for (int s = 0; s < kSets; ++s) {
            cs[s][j & 1] = mfma(a[s][j], hi, cs[s][j & 1]);
            cs[s][j & 1] = mfma(a[s][j], mid, cs[s][j & 1]);
            cs[s][j & 1] = mfma(a[s][j], lo, cs[s][j & 1]);
          }
        }
#pragma unroll
        for (int s = 0; s < kSets; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[t][s][0][r] = __builtin_fmaf(cs[s][0][r] + cs[s][1][r], scl[t], acc[t][s][0][r]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[t][0][j & 1] = mfma(a[0][j], mx_dword_to_bf16(w[t][j], scl[t]), acc[t][0][j & 1]);
      }
    }
  };
  auto fold = [&]() {
#pragma unroll
    for (int t = 0; t < kT; ++t)
#pragma unroll
      for (int s = 0; s < kSets; ++s) {
        f32x4_t v;
        if constexpr (kSplit) {
          // lanes 0..31 take their second block's rows from lane + 32
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = acc[t][s][0][r] + __shfl_xor(acc[t][s][0][r], 32);
        } else {
          v = acc[t][s][0] + acc[t][s][1];
        }
        tot[t][s] = tot[t][s] + v;
        acc[t][s][0] = acc[t][s][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
  };

  u32x4_t pair_sq[kT];   // NF4: the current chunk pair's absmax (taken before its refill)
  for (int c0 = 0; c0 < nchunks; c0 += kD) {
#pragma unroll
    for (int r = 0; r < kR; ++r) {
#pragma unroll
      for (int i = 0; i < kCpw; ++i) {
        const int slot = r * kCpw + i;
        const int c = c0 + slot;
        u32x4_t w[kT];
        float scl[kT];
        const bool kval = (unsigned)(c * 128 + q * 32) < (unsigned)K32;
#pragma unroll
        for (int t = 0; t < kT; ++t) {
          w[t] = wr[slot][t];
          if constexpr (kSplit) {
            // absmax block 2 c + q / 2: element 2 (c % 2) + q / 2 of the pair's
            // four; a lane past the end of K multiplies zeros by zero
            if ((slot & 1) == 0) {
              if constexpr (abs_block) {
                // floats 4 h .. 4 h + 3 of row nl (h = c / 2): lane (nl ssn + 4 h) / 4
                const int src = (nl * abs_row + 2 * c) & ~3;   // bytes: lane x 4
#pragma unroll
                for (int k = 0; k < 4; ++k)
                  pair_sq[t][k] = (unsigned)__builtin_amdgcn_ds_bpermute(src, (int)sgl[t][k]);
              } else {
                pair_sq[t] = sq[slot / 2][t];
              }
            }
            const u32x4_t v = pair_sq[t];
            const unsigned lo2 = (slot & 1) ? v[2] : v[0], hi2 = (slot & 1) ? v[3] : v[1];
            scl[t] = kval ? __uint_as_float(q >= 2 ? hi2 : lo2) : 0.f;
          } else {
            scl[t] = e8m0_to_f32(sb[slot][t]);
          }
        }
        issue(c + kD, slot);
        compute(c, w, scl);
        __builtin_amdgcn_sched_barrier(0);   // one chunk's registers at a time
      }
      fold();
    }
  }

  // ---- outputs
#pragma unroll
  for (int t = 0; t < kT; ++t)
#pragma unroll
    for (int s = 0; s < kSets; ++s) {
      const f32x4_t v = tot[t][s];
      if ((!kSplit || q < 2) && n[t] < p.N) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = (kSplit ? 8 * s : 0) + 4 * q + i;
          if (m < M) p.out[(int64_t)(r0 + m) * p.ldo + n[t]] = f32_to_bf16_bits(v[i]);
        }
      }
    }
  // the ring's last refills (past the end: zero-size offsets) are in flight
  __builtin_amdgcn_s_waitcnt(0);
}

// ------------------------------------------------- unit-streaming decode --
//
// k_decode_stream<kCpw, kR>: batched MXFP4 decode (groups of 2..16 rows) as
// a persistent walk over units. Workgroup (x, g) takes a contiguous range
// of group g's units (32 weight rows each); its eight waves split each
// unit's K chunks exactly as k_decode_fwd does (wave w: chunks w kCpw ..
// w kCpw + kCpw - 1, one round) and the unit's partial tiles are reduced
// through LDS in wave order, so the outputs are k_decode_fwd's bits. What
// changes is the memory side:
//   * the group's activation rows are staged into LDS once per workgroup,
//     not loaded again by every unit (at 9..16 rows k_decode_fwd loads them
//     into registers per unit: as many load requests as the weights);
//   * each wave keeps the weight and scale loads of kR units in flight in a
//     register ring (one workgroup per CU, two waves per SIMD)
//     and refills a slot as soon as its unit's MFMAs have consumed it, so
//     the decode, the reduction and the stores of one unit overlap the
//     loads of the next ones.
// (An NF4 split-codebook form of this walk, one or two teams of eight
// waves, measured 3-8 % slower than k_decode_fwd at Qwen3 batch 8..16: its
// per-byte LDS lookups need the per-unit kernel's four waves per SIMD.)
// kLdsScales: a unit's scale bytes (32 contiguous rows, at most 3 KiB) come
// in as three coalesced 16-byte-per-lane loads by waves 0..2 and reach the
// other waves through an LDS ring, where each wave otherwise loads its own
// bytes, one per lane and 16 rows per load. The bytes are the same; the
// memory side sees 45 requests per unit instead of 768: measured on MI355X
// (GPT-OSS gate_up), the per-lane byte loads cost 15 % of the kernel's time
// against a build without scale loads.
// LDS: [activations, padded as in decode_unit][zero block][partial tiles:
// 8 waves x 2 tiles x 64 lanes x 16 B][kLdsScales: kR x 3 KiB of scales].
template <int kCpw, int kR, bool kLdsScales>
__global__ void __launch_bounds__(512, 1)
    k_decode_stream(const FwdArgs p, const int upg, const int per_wg) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int kW = 8, kT = 2;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int q = lane >> 4;
  const int g = (int)blockIdx.y;
  const int u0 = (int)blockIdx.x * per_wg;
  const int n_units = (upg - u0 < per_wg ? upg - u0 : per_wg);
  if (n_units <= 0) return;

  int e32, ro_a, ro_b;
  asm volatile(
      "s_load_dword %0, %3, 0x0\n\t"
      "s_load_dword %1, %4, 0x0\n\t"
      "s_load_dword %2, %5, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(e32), "=&s"(ro_a), "=&s"(ro_b)
      : "s"(p.eids + g), "s"(p.row_off + (g << p.ro_shift)),
        "s"(p.row_off + (g << p.ro_shift) + 1)
      : "memory");
  const int64_t e = e32;
  const int r0 = ro_a;
  const int M = ro_b - ro_a;
  if (M <= 0) return;
  const int K32 = (int)p.K;
  const int kslices = K32 >> 3;
  const int pieces = M * kslices;
  const int zero_off = (pieces + (kslices >> 2) + 1) * 16;
  const int red_off = zero_off + 64;
  const int sc_off = red_off + kW * kT * 64 * 16;
  const int c0 = wave * kCpw;

  // ---- the first eight activation pieces per thread go out before the
  // ring's loads (the staging then waits for them alone)
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + (int64_t)r0 * p.lda, (int64_t)M * p.lda * 2);
  u32x4_t av[8];
  auto stage_load = [&](int base) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int pc = base + j * 512 + (int)threadIdx.x;
      const int m = pc / kslices, sl = pc - m * kslices;
      av[j] = buf_load16(ra, oob_unless(pc < pieces, (int)((int64_t)m * p.lda * 2) + sl * 16));
    }
  };
  auto stage_store = [&](int base) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int pc = base + j * 512 + (int)threadIdx.x;
      if (pc < pieces) {
        const int m = pc / kslices, sl = pc - m * kslices;
        *reinterpret_cast<u32x4_t*>(smem + (sl * M + m + (sl >> 2)) * 16) = av[j];
      }
    }
  };
  stage_load(0);

  // ---- the ring's first kR units
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + e * p.sbe, p.N * p.sbn);
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(static_cast<const uint8_t*>(p.S) + e * p.sse, p.N * p.ssn);
  u32x4_t wr[kR][kCpw][kT];
  // (bytes: held as 32-bit values they get re-masked at the loop's back
  // edge, and the mask waits for the newest loads)
  uint8_t sb[kR][kCpw][kT];
  u32x4_t sg[kR];   // kLdsScales, waves 0..2: 1 KiB each of the unit's scale block
  auto issue = [&](int u, int slot) {
    // units past the workgroup's range load zeros (offsets past every resource)
    const bool live = u < n_units;
    if constexpr (kLdsScales) {
      // ahead of the unit's weights, so waiting for it waits for no weights
      // of its own unit
      if (wave < 3)
        sg[slot] = buf_load16(rs, oob_unless(live, (int)((int64_t)(u0 + u) * 32 * p.ssn) +
                                                       wave * 1024 + lane * 16));
    }
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      const int64_t n = (int64_t)(u0 + u) * (16 * kT) + t * 16 + nl;
      const bool nok = live && n < p.N;
      const int b_row = (int)(n * p.sbn), s_row = (int)(n * p.ssn);
#pragma unroll
      for (int i = 0; i < kCpw; ++i) {
        const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
        const bool kval = nok && kseg < (unsigned)K32;
        wr[slot][i][t] = buf_load16(rb, oob_unless(kval, b_row + (int)(kseg >> 1)));
        if constexpr (!kLdsScales)
          sb[slot][i][t] = buf_load1(rs, oob_unless(kval, s_row + (int)(kseg >> 5)));
      }
    }
  };
  // the scale block of the unit in ring slot `slot` into its LDS slot
  auto put_scales = [&](int slot) {
    if constexpr (kLdsScales) {
      if (wave < 3)
        *reinterpret_cast<u32x4_t*>(smem + sc_off + slot * 3072 + wave * 1024 + lane * 16) =
            sg[slot];
    }
  };
#pragma unroll
  for (int r = 0; r < kR; ++r) issue(r, r);

  // ---- activations into LDS, once
  stage_store(0);
  for (int base = 8 * 512; base < pieces; base += 8 * 512) {
    stage_load(base);
    stage_store(base);
  }
  if (threadIdx.x < 4)
    *reinterpret_cast<u32x4_t*>(smem + zero_off + threadIdx.x * 16) = u32x4_t{0u, 0u, 0u, 0u};
  put_scales(0);
  lds_barrier();   // the ring's weight loads stay in flight

  f32x4_t* s_red = reinterpret_cast<f32x4_t*>(smem + red_off);   // [wave][t][64]
  // the A operands of the wave's chunks: the same for every unit (token nl)
  auto a_operand = [&](int i, int j) {
    const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
    const int sl = (int)(kseg >> 3) + j;
    const int off = (kseg < (unsigned)K32 && nl < M) ? (sl * M + nl + (sl >> 2)) * 16 : zero_off;
    return *reinterpret_cast<const u32x4_t*>(smem + off);
  };

  auto walk_unit = [&](const int u, auto slot_c) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    // ---- unit u: this wave's run, from ring slot `slot`, in k_decode_fwd's
    // order (two accumulators per tile, alternate k-slices)
    f32x4_t acc[kT][2];
#pragma unroll
    for (int t = 0; t < kT; ++t) acc[t][0] = acc[t][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kCpw; ++i) {
      u32x4_t a[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = a_operand(i, j);
#pragma unroll
      for (int t = 0; t < kT; ++t) {
        unsigned sbyte;
        if constexpr (kLdsScales) {
          // a chunk past K reads scale 0, as the direct load does
          const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
          const int off = sc_off + slot * 3072 + (t * 16 + nl) * (int)p.ssn + (int)(kseg >> 5);
          sbyte = kseg < (unsigned)K32 ? *reinterpret_cast<const uint8_t*>(smem + off) : 0u;
        } else {
          sbyte = sb[slot][i][t];
        }
        const float sc = e8m0_to_f32(sbyte);
        u32x4_t b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = mx_dword_to_bf16(wr[slot][i][t][j], sc);
        acc[t][0] = mfma(a[0], b[0], acc[t][0]);
        acc[t][1] = mfma(a[1], b[1], acc[t][1]);
        acc[t][0] = mfma(a[2], b[2], acc[t][0]);
        acc[t][1] = mfma(a[3], b[3], acc[t][1]);
      }
    }
    // the slot's registers are consumed: refill them with unit u + kR (the
    // loads write the same registers, so no copy waits for them)
    issue(u + kR, slot);
    // ---- the unit's tiles over the waves, in wave order
    lds_barrier();   // the previous unit's partials have been read
    // unit u + 1's scales into the LDS slot unit u + 1 - kR read (every
    // wave is past that unit); visible after the next barrier
    put_scales(slot + 1 < kR ? slot + 1 : 0);
#pragma unroll
    for (int t = 0; t < kT; ++t) s_red[(wave * kT + t) * 64 + lane] = acc[t][0] + acc[t][1];
    lds_barrier();
    if (wave < kT) {
      const int t = wave;
      const f32x4_t* r = s_red + t * 64 + lane;
      f32x4_t v = r[0];
#pragma unroll
      for (int w2 = 1; w2 < kW; ++w2) v = v + r[w2 * kT * 64];
      const int64_t n = (int64_t)(u0 + u) * (16 * kT) + t * 16 + nl;
      if (n < p.N) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 4 * q + i;
          if (m < M) p.out[(int64_t)(r0 + m) * p.ldo + n] = f32_to_bf16_bits(v[i]);
        }
      }
    }
  };
  // Whole turns of the ring, then the last n_units % kR units. The loop has
  // one exit, at the end of a turn: an exit in mid-turn is joined to the
  // back edge, and the wait counts at the top of the turn then assume that
  // the first slot's refill is the newest load, which drains the ring there.
  int ub = 0;
  auto turn = [&](auto slot_c) {
    walk_unit(ub + decltype(slot_c)::value, slot_c);
    return true;
  };
  auto tail = [&](auto slot_c) {
    if (ub + decltype(slot_c)::value >= n_units) return false;
    walk_unit(ub + decltype(slot_c)::value, slot_c);
    return true;
  };
  for (; ub + kR <= n_units; ub += kR) StepUnroll<0, kR>::run(turn);
  StepUnroll<0, kR>::run(tail);
  // the ring's last refills (past the range: zero-size offsets) are in flight
  __builtin_amdgcn_s_waitcnt(0);
}

// k_decode_stream_nf4<kR, kT>: the unit walk for NF4 groups of 2..8 rows
// (split codebook, one row set, two chunks per wave: 768 < K <= 2048), units
// of 16 kT weight rows. Two teams of eight waves per workgroup (four waves
// per SIMD, as k_decode_fwd runs), team t on units t, t + 2, ... of the
// range. The split table is built and the group's activation rows are
// staged into LDS once per workgroup, where k_decode_fwd builds the table
// and loads the activations (into registers) once per unit; each slice's
// lookups and MFMAs run one at a time (sched_barrier) to stay within 128
// VGPRs. Same chunk split per wave and reduction order as k_decode_fwd: the
// same bits. The split decode keeps the LDS busy (16 bytes read per weight
// byte), so deeper load rings do not pay here: measured on MI355X (Qwen3
// gate_up), one unit in flight per team, 16-row units: batch 8 33.1 -> 31.8
// us, batch 16 50.1 -> 47.5..48.7 us; rings of two or three units and
// 32-row units ran slower.
template <int kR, int kT>
__global__ void __launch_bounds__(1024, 1)
    k_decode_stream_nf4(const FwdArgs p, const int upg, const int per_wg) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int kW = 8, kCpw = 2, kTeams = 2, kThreads = 1024;
  const int lut = nf4_lut_lane();
  __builtin_amdgcn_sched_barrier(0);
  const int lane = threadIdx.x & 63;
  const int wave = (threadIdx.x >> 6) & (kW - 1);
  const int team = (int)threadIdx.x >> 9;
  const int nl = lane & 15;
  const int q = lane >> 4;
  const int g = (int)blockIdx.y;
  const int u0 = (int)blockIdx.x * per_wg;
  const int n_units = (upg - u0 < per_wg ? upg - u0 : per_wg);
  if (n_units <= 0) return;
  int e32, ro_a, ro_b;
  asm volatile(
      "s_load_dword %0, %3, 0x0\n\t"
      "s_load_dword %1, %4, 0x0\n\t"
      "s_load_dword %2, %5, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(e32), "=&s"(ro_a), "=&s"(ro_b)
      : "s"(p.eids + g), "s"(p.row_off + (g << p.ro_shift)),
        "s"(p.row_off + (g << p.ro_shift) + 1)
      : "memory");
  const int64_t e = e32;
  const int r0 = ro_a;
  const int M = ro_b - ro_a;
  if (M <= 0) return;
  const int K32 = (int)p.K;
  const int kslices = K32 >> 3;
  const int pieces = M * kslices;
  const int a_base = kSplitTabBytes;
  const int zero_off = a_base + (pieces + (kslices >> 2) + 1) * 16;
  const int red_off = zero_off + 64 + team * (kW * kT * 64 * 16);
  const int c0 = wave * kCpw;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + (int64_t)r0 * p.lda, (int64_t)M * p.lda * 2);
  u32x4_t av[4];
  auto stage_load = [&](int base) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pc = base + j * kThreads + (int)threadIdx.x;
      const int m = pc / kslices, sl = pc - m * kslices;
      av[j] = buf_load16(ra, oob_unless(pc < pieces, (int)((int64_t)m * p.lda * 2) + sl * 16));
    }
  };
  auto stage_store = [&](int base) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pc = base + j * kThreads + (int)threadIdx.x;
      if (pc < pieces) {
        const int m = pc / kslices, sl = pc - m * kslices;
        *reinterpret_cast<u32x4_t*>(smem + a_base + (sl * M + m + (sl >> 2)) * 16) = av[j];
      }
    }
  };
  stage_load(0);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + e * p.sbe, p.N * p.sbn);
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(static_cast<const char*>(p.S) + e * p.sse * 4, p.N * p.ssn * 4);
  u32x4_t wr[kR][kCpw][kT];
  u32x4_t sq[kR][kT];
  auto issue = [&](int j, int slot) {
    const int ul = j * kTeams + team;
    const bool live = ul < n_units;
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      const int64_t n = (int64_t)(u0 + ul) * (16 * kT) + t * 16 + nl;
      const bool nok = live && n < p.N;
      const int b_row = (int)(n * p.sbn), s_row = (int)(n * p.ssn * 4);
#pragma unroll
      for (int i = 0; i < kCpw; ++i) {
        const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
        wr[slot][i][t] =
            buf_load16(rb, oob_unless(nok && kseg < (unsigned)K32, b_row + (int)(kseg >> 1)));
      }
      sq[slot][t] = buf_load16(rs, oob_unless(nok && (unsigned)(c0 * 128) < (unsigned)K32,
                                              s_row + c0 * 8));
    }
  };
#pragma unroll
  for (int r = 0; r < kR; ++r) issue(r, r);
  stage_store(0);
  for (int base = 4 * kThreads; base < pieces; base += 4 * kThreads) {
    stage_load(base);
    stage_store(base);
  }
  if (threadIdx.x < 4)
    *reinterpret_cast<u32x4_t*>(smem + zero_off + threadIdx.x * 16) = u32x4_t{0u, 0u, 0u, 0u};
  if (threadIdx.x < 512) init_split_table(smem, lut);
  lds_barrier();

  const bool blk_lane = (nl < 8) == (q < 2);
  const int tok = nl & 7;
  const unsigned lane_off = (unsigned)(uintptr_t)smem | (unsigned)(lane & (kSplitCols - 1)) * 16u;
  f32x4_t* s_red = reinterpret_cast<f32x4_t*>(smem + red_off);
  const int n_steps = (n_units + kTeams - 1) / kTeams;
  for (int jb = 0; jb < n_steps; jb += kR) {
#pragma unroll
    for (int slot = 0; slot < kR; ++slot) {
      const int j = jb + slot;
      if (j >= n_steps) break;
      const int ul = j * kTeams + team;
      f32x4_t acc[kT];
#pragma unroll
      for (int t = 0; t < kT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < kCpw; ++i) {
        const unsigned kseg = (unsigned)((c0 + i) * 128 + q * 32);
        const bool aval = kseg < (unsigned)K32 && blk_lane && tok < M;
#pragma unroll
        for (int t = 0; t < kT; ++t) {
          const int idx = 2 * i + (q >> 1);
          const u32x4_t v = sq[slot][t];
          const float am = __uint_as_float(idx == 0 ? v[0] : idx == 1 ? v[1] : idx == 2 ? v[2] : v[3]);
          f32x4_t c[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int sl = (int)(kseg >> 3) + jj;
            const u32x4_t a = *reinterpret_cast<const u32x4_t*>(
                smem + (aval ? a_base + (sl * M + tok + (sl >> 2)) * 16 : zero_off));
            u32x4_t hi, mid, lo;
            split_lookup(wr[slot][i][t][jj], lane_off, hi, mid, lo);
            c[jj & 1] = mfma(a, hi, c[jj & 1]);
            c[jj & 1] = mfma(a, mid, c[jj & 1]);
            c[jj & 1] = mfma(a, lo, c[jj & 1]);
            __builtin_amdgcn_sched_barrier(0);   // one slice's registers at a time
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(c[0][r] + c[1][r], am, acc[t][r]);
        }
      }
      issue(j + kR, slot);
      lds_barrier();
#pragma unroll
      for (int t = 0; t < kT; ++t) s_red[(wave * kT + t) * 64 + lane] = acc[t];
      lds_barrier();
      if (wave < kT && ul < n_units) {
        const int t = wave;
        const f32x4_t* r = s_red + t * 64 + lane;
        f32x4_t v = r[0] + r[32];
#pragma unroll
        for (int w2 = 1; w2 < kW; ++w2) v = v + (r[w2 * kT * 64] + r[w2 * kT * 64 + 32]);
        const int64_t n = (int64_t)(u0 + ul) * (16 * kT) + t * 16 + nl;
        if (q < 2 && n < p.N) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * q + i;
            if (m < M) p.out[(int64_t)(r0 + m) * p.ldo + n] = f32_to_bf16_bits(v[i]);
          }
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
}

// ------------------------------------------------------------ fused FFN --
//
// gate_up -> silu(gate) * up -> down for groups of at most 16 rows, in one
// launch. Workgroups [0, G * H / 16) are gate/up units, the rest are down
// units (G * ceil(N_dn / 32)), both in group-major order. A down unit only
// waits on gate/up units, which have smaller ids; workgroups are dispatched
// in id order and gate/up units never wait, so the wait always ends. A
// bounded spin backs this up: a down unit that polls `spin_limit` times
// without seeing its flags sets the error word, writes NaN into its output
// rows instead of a result, and exits.
//
// Hand-off without cache maintenance or atomics: a gate/up unit writes its
// 16 columns of h (bf16, [T, ldh]) with device-scope stores, waits for them
// to complete, and then writes this call's epoch (a nonzero per-call value)
// into its flag in the private flag row of every down unit of its group
// (device-scope stores). A down unit issues its weight loads, polls its own
// row with one device-scope vector load until every flag holds the epoch,
// reads h with device-scope loads, and clears its row: it is the row's only
// reader, so the words are zero again for the next call (and for graph
// replays) without any counting. A flag left behind by a call that timed
// out holds an older epoch, which no later call's down unit accepts.
// Release/acquire fences would write back or invalidate whole L2 caches per
// unit, and same-address atomics serialise at about 0.1 us each; both cost
// more than the launch this saves.
//
// Sync words (u32, device memory, zero before the first call): [0] error
// flag (sticky: set by a timed-out down unit, cleared only by the caller),
// then G * ceil(N_dn / 32) rows of H / 16 flags from word kFfnFlagBase.
// Calls that overlap on one sync buffer race.
constexpr int kFfnSpinLimit = 1 << 22;   // default polls before a down unit gives up
constexpr int kFfnMaxDynLds = 160 * 1024;

template <int CPW1, int CPW2, int kAPieces, int kSets>
__global__ void __launch_bounds__(512, 4) k_ffn_decode(const FwdArgs gu, const FwdArgs dn,
                                                       const int64_t H, uint32_t* sync,
                                                       const uint32_t epoch,
                                                       const int spin_limit) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int lut = nf4_lut_lane();
  __builtin_amdgcn_sched_barrier(0);
  // every gate/up unit (group-major) comes before every down unit: the
  // gate/up phase runs at full width, and a down unit that starts early
  // streams its weights while the last gate/up units finish
  const int64_t gu_per_group = H / 16;
  const int64_t dn_per_group = (dn.N + 31) / 32;
  const int64_t gu_units = (int64_t)gu.G * gu_per_group;
  const int64_t u = blockIdx.x;
  if (u < gu_units) {
    // unit counts stay below 2^31 (the launch checks): 32-bit division
    const int gg = (int)((uint32_t)u / (uint32_t)gu_per_group);
    decode_unit<kNF4, CPW1, 2, 8, kAPieces, kFfnGu, kSets>(
        gu, gg, u - (int64_t)gg * gu_per_group, smem, lut, H, dn.N, sync, epoch, NoWait{});
    return;
  }
  const int64_t d = u - gu_units;
  const int g = (int)((uint32_t)d / (uint32_t)dn_per_group);
  const int32_t* ro = dn.row_off ? dn.row_off + (g << dn.ro_shift) : nullptr;
  const int M = ro ? ro[1] - ro[0] : 1;
  if (M <= 0) return;                   // empty group: no gate/up unit sets its flags
  uint32_t* row = sync + kFfnFlagBase + d * gu_per_group;
  auto wait_h = [&](int* status) {
    if (threadIdx.x < 64) {             // wave 0 polls the row, 64 flags per load
      const int lane = threadIdx.x;
      int spins = 0;
      bool timed_out = false;
      while (true) {
        bool all = true;
        for (int64_t j = lane; j < gu_per_group; j += 64)
          all &= __hip_atomic_load(row + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
        if (__builtin_amdgcn_ballot_w64(!all) == 0) break;
        if (++spins > spin_limit) {     // not expected: flag it, poison the outputs
          timed_out = true;
          if (lane == 0)
            __hip_atomic_store(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      for (int64_t j = lane; j < gu_per_group; j += 64)   // this row's only reader
        __hip_atomic_store(row + j, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane == 0) *status = timed_out ? 1 : 0;
    }
    // no wave issues an h load before wave 0 has seen every flag (the weight
    // loads already in flight need not land first); the status word is
    // visible to every wave after the barrier
    __syncthreads();
  };
  decode_unit<kNF4, CPW2, 2, 8, kAPieces, kFfnDn, kSets>(dn, g, d - (int64_t)g * dn_per_group, smem,
                                                         lut, 0, 0, sync, 0u, wait_h);
}

// Elementwise silu-multiply for the unfused path (and groups too large for
// the fused decode kernel): h[t, j] = bf16(silu_locked(gu[t, j]) * gu[t, H + j]),
// gu bf16 [T, ldg], h bf16 [T, ldh]. Eight columns per thread.
template <class Idx>
__global__ void __launch_bounds__(256) k_silu_mul(const uint16_t* __restrict__ gu, int64_t ldg,
                                                  uint16_t* __restrict__ h, int64_t ldh, Idx T,
                                                  Idx H) {
  const Idx vec = H / 8, total = T * vec;
  for (Idx i = (Idx)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (Idx)gridDim.x * blockDim.x) {
    const int64_t t = i / vec, c = (i - (Idx)t * vec) * 8;
    const u32x4_t gv = *reinterpret_cast<const u32x4_t*>(gu + t * ldg + c);
    const u32x4_t uv = *reinterpret_cast<const u32x4_t*>(gu + t * ldg + H + c);
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = __uint_as_float(gv[j] << 16), g1 = __uint_as_float(gv[j] & 0xFFFF0000u);
      const float u0 = __uint_as_float(uv[j] << 16), u1 = __uint_as_float(uv[j] & 0xFFFF0000u);
      o[j] = (uint32_t)f32_to_bf16_bits(silu_locked(g0) * u0) |
             ((uint32_t)f32_to_bf16_bits(silu_locked(g1) * u1) << 16);
    }
    *reinterpret_cast<u32x4_t*>(h + t * ldh + c) = o;
  }
}

// ============================================================ tiled GEMM ==

constexpr int kLdsRow = 64 + 8;   // bf16 elements per staged row (16 B pad)
constexpr int kBN = 128;          // forward n-tile
constexpr int kThreads = 256;

// Stage one 64-wide k-step of BM activation rows into LDS (zero-filled
// outside [rows) x [K)). Each thread moves 16 B per pass.
template <int BM>
__device__ __forceinline__ void load_a_tile(u32x4_t (&r)[(BM * 8 + kThreads - 1) / kThreads],
                                            const uint16_t* a, int64_t lda, int64_t row0,
                                            int rows, int64_t k0, int64_t K) {
  constexpr int P = (BM * 8 + kThreads - 1) / kThreads;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    const int rr = idx >> 3, kc = (idx & 7) * 8;
    const bool ok = idx < BM * 8 && rr < rows && k0 + kc < K;
    r[i] = ok ? load_a8(a + (row0 + rr) * lda + k0 + kc) : u32x4_t{0u, 0u, 0u, 0u};
  }
}

template <int BM>
__device__ __forceinline__ void store_a_tile(const u32x4_t (&r)[(BM * 8 + kThreads - 1) / kThreads],
                                             uint16_t* lds) {
  constexpr int P = (BM * 8 + kThreads - 1) / kThreads;
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    if (idx < BM * 8) {
      const int rr = idx >> 3, kc = (idx & 7) * 8;
      *reinterpret_cast<u32x4_t*>(lds + rr * kLdsRow + kc) = r[i];
    }
  }
}

// Forward weight tile: kBN rows x 64 k = 32 packed bytes per row; thread t
// owns row t / 2, bytes [16 (t % 2), +16) = 32 elements (one MX block, half an
// NF4 block), so it needs exactly one scale.
template <int FMT>
struct BTileRegs {
  u32x4_t w;
  float s;
};

template <int FMT>
__device__ __forceinline__ void load_b_fwd(BTileRegs<FMT>& r, const FwdArgs& p, int64_t e,
                                           int64_t n0, int64_t k0) {
  const int rr = threadIdx.x >> 1, half = threadIdx.x & 1;
  const int64_t n = n0 + rr;
  const int64_t k = k0 + half * 32;
  if (n < p.N && k < p.K) {
    r.w = *reinterpret_cast<const u32x4_t*>(p.B + e * p.sbe + n * p.sbn + (k >> 1));
    r.s = load_scale<FMT>(p, e, n, k);
  } else {
    r.w = u32x4_t{0u, 0u, 0u, 0u};
    r.s = 0.0f;
  }
}

template <int FMT>
__device__ __forceinline__ void store_b_fwd(const BTileRegs<FMT>& r, const float2* tab,
                                            uint16_t* lds) {
  const int rr = threadIdx.x >> 1, half = threadIdx.x & 1;
  const unsigned lane_off = (unsigned)(threadIdx.x & 31) * 8u;
  uint16_t* dst = lds + rr * kLdsRow + half * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x4_t v;
    if constexpr (FMT == kNF4) v = nf4_dword_to_bf16(tab, r.w[i], lane_off, r.s);
    else v = mx_dword_to_bf16(r.w[i], r.s);
    *reinterpret_cast<u32x4_t*>(dst + 8 * i) = v;
  }
}

// fp32-weight form (the reference's VARIANT 1, kernel/nf4_grouped.py:446-452,
// which takes the fp32 products LUT x absmax into the dot): each fp32 weight
// w = LUT * absmax (one rounding) splits into hi = bf16(w) and lo =
// bf16(w - hi) (w - hi is exact in fp32), so hi + lo carries w to within
// 2^-17 of its magnitude, and two MFMAs (hi, then lo) add both parts.
template <int FMT>
__device__ __forceinline__ void store_b_fwd_hilo(const BTileRegs<FMT>& r, const float2* tab,
                                                 uint16_t* lds_hi, uint16_t* lds_lo) {
  static_assert(FMT == kNF4, "MXFP4 weights are exact in bf16");
  const int rr = threadIdx.x >> 1, half = threadIdx.x & 1;
  const unsigned lane_off = (unsigned)(threadIdx.x & 31) * 8u;
  const int off = rr * kLdsRow + half * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x4_t vh, vl;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const unsigned addr = __builtin_amdgcn_perm(r.w[i], lane_off, 0x0C0C0000u | ((4u + b) << 8));
      const float2 pr = *reinterpret_cast<const float2*>(reinterpret_cast<const char*>(tab) + addr);
      const float w0 = pr.x * r.s, w1 = pr.y * r.s;
      const float h0 = bf16_round(w0), h1 = bf16_round(w1);
      vh[b] = bf16x2_bits(h0, h1);
      vl[b] = bf16x2_bits(w0 - h0, w1 - h1);
    }
    *reinterpret_cast<u32x4_t*>(lds_hi + off + 8 * i) = vh;
    *reinterpret_cast<u32x4_t*>(lds_lo + off + 8 * i) = vl;
  }
}

// Waves: WM x WN = 4. Wave tile (BM / WM) x (BN / WN) in 16 x 16 MFMA tiles.
template <int BM> struct WaveGrid { static constexpr int WM = BM >= 64 ? 2 : 1; };

// HL: the fp32-weight form (store_b_fwd_hilo), NF4 only, BM <= 64 (LDS).
template <int FMT, int BM, bool HL = false>
__global__ void __launch_bounds__(kThreads, 1) k_gemm_fwd(const FwdArgs p) {
  static_assert(!HL || (FMT == kNF4 && BM <= 64), "fp32-weight tiles: NF4, at most 64 rows");
  constexpr int WM = WaveGrid<BM>::WM, WN = 4 / WM;
  constexpr int MT = BM / WM / 16, NT = kBN / WN / 16;
  constexpr int AP = (BM * 8 + kThreads - 1) / kThreads;
  __shared__ float2 s_tab[FMT == kNF4 ? kPairEntries : 1];
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t s_b[2][kBN * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t s_bl[HL ? 2 : 1][HL ? kBN * kLdsRow : 8];
  if constexpr (FMT == kNF4) init_pair_table(s_tab, nf4_lut_lane());

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l16 = lane & 15, q = lane >> 4;
  const int64_t n_tiles = (p.N + kBN - 1) / kBN;
  const int64_t total = (int64_t)p.n_mtiles * n_tiles;
  const int64_t ksteps = (p.K + 63) >> 6;

  for (int64_t t = blockIdx.x; t < total; t += gridDim.x) {
    const int mt = (int)(t / n_tiles);
    const int64_t n0 = (t - (int64_t)mt * n_tiles) * kBN;
    const int64_t row0 = p.t_row0[mt];
    const int rows = p.t_rows[mt];
    const int64_t e = p.eids[p.t_group[mt]];

    u32x4_t areg[AP];
    BTileRegs<FMT> breg;
    __syncthreads();  // previous tile's LDS readers are done (and table ready)
    load_a_tile<BM>(areg, p.a, p.lda, row0, rows, 0, p.K);
    load_b_fwd<FMT>(breg, p, e, n0, 0);
    store_a_tile<BM>(areg, s_a[0]);
    if constexpr (HL) store_b_fwd_hilo<FMT>(breg, s_tab, s_b[0], s_bl[0]);
    else store_b_fwd<FMT>(breg, s_tab, s_b[0]);
    __syncthreads();

    f32x4_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int64_t ks = 0; ks < ksteps; ++ks) {
      const int cur = (int)(ks & 1);
      const bool more = ks + 1 < ksteps;
      if (more) {
        load_a_tile<BM>(areg, p.a, p.lda, row0, rows, (ks + 1) * 64, p.K);
        load_b_fwd<FMT>(breg, p, e, n0, (ks + 1) * 64);
      }
      const uint16_t* la = s_a[cur];
      const uint16_t* lb = s_b[cur];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u32x4_t bop[NT], bol[HL ? NT : 1];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int bo = ((wn * NT + j) * 16 + l16) * kLdsRow + kk * 32 + q * 8;
          bop[j] = *reinterpret_cast<const u32x4_t*>(lb + bo);
          if constexpr (HL) bol[j] = *reinterpret_cast<const u32x4_t*>(&s_bl[cur][bo]);
        }
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const u32x4_t aop = *reinterpret_cast<const u32x4_t*>(
              la + ((wm * MT + i) * 16 + l16) * kLdsRow + kk * 32 + q * 8);
#pragma unroll
          for (int j = 0; j < NT; ++j) {
            acc[i][j] = mfma(aop, bop[j], acc[i][j]);
            if constexpr (HL) acc[i][j] = mfma(aop, bol[j], acc[i][j]);
          }
        }
      }
      if (more) {
        store_a_tile<BM>(areg, s_a[cur ^ 1]);
        if constexpr (HL) store_b_fwd_hilo<FMT>(breg, s_tab, s_b[cur ^ 1], s_bl[cur ^ 1]);
        else store_b_fwd<FMT>(breg, s_tab, s_b[cur ^ 1]);
      }
      __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int64_t n = n0 + (wn * NT + j) * 16 + l16;
        if (n >= p.N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = (wm * MT + i) * 16 + 4 * q + r;
          if (m < rows) p.out[(row0 + m) * p.ldo + n] = f32_to_bf16_bits(acc[i][j][r]);
        }
      }
    }
  }
}

// ============================================================== prefill ==
//
// Tiled forward for groups larger than the decode path takes. Tile: 128 rows
// of one group x 256 weight rows (n); four waves, wave w owns the 64 weight
// rows [64 w, 64 w + 64) for all 128 activation rows, so no weight element is
// decoded twice. K advances in steps of 64.
//
//   * weights: each lane loads 8 packed bytes (16 k values) per 16-row
//     n-subtile and step straight into registers and decodes them into two
//     MFMA operands (the weights are MFMA operand A, so the accumulator holds
//     out^T and a lane ends with 4 consecutive output columns of one row);
//   * activations: a ring of three 16 KiB LDS stages filled by buffer loads
//     that write LDS directly (no VGPR round trip). A stage holds 128 rows x
//     64 k; 16-byte slots are swizzled per row (pf_swz) so the 16-byte
//     operand reads of a wave run at the full 256 B per clock;
//   * one flat software pipeline over (tile, k-step) pairs of the workgroup's
//     whole tile list: the loads of step f + 2 are in flight while step f
//     computes, across tile boundaries;
//   * tiles: a persistent grid; the tile list (m-tile major, n-tile minor, so
//     a group's tiles are adjacent) is cut into eight contiguous ranges, one
//     per XCD (workgroup b runs on XCD b % 8), so the tiles an XCD runs at
//     the same time share weights and activations in that XCD's L2.
//
// Every vector-memory instruction of a step is counted: kPfGroupLoads per
// step and wave. The waits on the LDS stages are explicit s_waitcnt
// immediates computed from that count (stores only add to the count, which
// makes a wait stricter, never looser).
constexpr int kPfBM = 128;
constexpr int kPfBN = 256;
constexpr int kPfBK = 64;
constexpr int kPfStage = kPfBM * kPfBK * 2; // bytes per LDS stage

// s_waitcnt with vmcnt(n) and lgkmcnt(0), expcnt untouched (gfx9 encoding).
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (0 << 8) | ((n >> 4) << 14));
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Values the kernel knows to be wave-uniform but the compiler may not (it
// would otherwise keep buffer descriptors in VGPRs and loop over lanes).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <class T>
__device__ __forceinline__ void* uniform_ptr(const T* ptr) {
  const uint64_t v = reinterpret_cast<uint64_t>(ptr);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return reinterpret_cast<void*>(lo | (hi << 32));
}
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// LDS slot swizzle of a staged activation row: 16-byte slot s of row m lives
// at slot s ^ pf_swz(m % 16). Over the 16 rows one operand read touches this
// spreads the 16-byte pieces across all 64 banks.
__device__ __forceinline__ int pf_swz(int m16) { return (m16 ^ (m16 >> 3)) & 7; }

struct PfTile {
  int row0, rows, e, n0;
};


template <int FMT, int kS>
__global__ void __launch_bounds__(512, 2)
    k_prefill(const FwdArgs p, const int32_t* __restrict__ t_row0,
              const int32_t* __restrict__ t_rows, const int32_t* __restrict__ t_group,
              const int32_t* __restrict__ eids, uint16_t* __restrict__ out) {
  static_assert(kS == 4, "ring depth: even, and four 16 KiB stages fill the low 64 KiB");
  constexpr int kWaves = 8;
  constexpr int kWaveCols = kPfBN / kWaves;          // 32: one 32 x 32 MFMA column block
  constexpr int kAPieces = kPfStage / 1024 / kWaves; // LDS-direct loads per wave and step
  constexpr int kRowsPerWave = kPfBM / kWaves;
  constexpr int kGroupLoads = kAPieces + 2;          // + weights + scale
  constexpr int kMT = kPfBM / 32;                    // activation subtiles of 32 rows
  static_assert(kWaveCols == 32, "one weight subtile per wave");
  // one LDS object per stage, so the compiler can tell the stages apart when
  // it places the waits for the direct-to-LDS loads
  __shared__ __attribute__((aligned(16))) char s_a0[kPfStage];
  __shared__ __attribute__((aligned(16))) char s_a1[kPfStage];
  __shared__ __attribute__((aligned(16))) char s_a2[kPfStage];
  __shared__ __attribute__((aligned(16))) char s_a3[kPfStage];
  // NF4 pair table: dynamic LDS, which follows the 64 KiB of static stages, so
  // it starts at 0x10000 and the stages keep addresses an instruction's
  // 16-bit offset field can hold.
  extern __shared__ __attribute__((aligned(16))) float2 s_tab[];
  auto stage_of = [&](auto RI) -> char* {
    constexpr int r = decltype(RI)::value;
    if constexpr (r == 0) return s_a0;
    else if constexpr (r == 1) return s_a1;
    else if constexpr (r == 2) return s_a2;
    else return s_a3;
  };
  const int lut = FMT == kNF4 ? nf4_lut_lane() : 0;
  __builtin_amdgcn_sched_barrier(0);
  const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  // table base (0x10000: byte 2) | lane column; nf4_dword_to_bf16_at takes
  // byte 2 of this register as address byte 2
  const unsigned tab_base = (unsigned)(uintptr_t)s_tab;
  const unsigned lane_off = tab_base | (unsigned)(lane & 31) * 8u;
  const char* lds0 = reinterpret_cast<const char*>(s_tab) - tab_base;
  constexpr int kScaleBytes = FMT == kNF4 ? 4 : 1;

  // ---- this workgroup's tiles
  const int n_tiles = (int)((p.N + kPfBN - 1) / kPfBN);
  const int64_t total = (int64_t)p.n_mtiles * n_tiles;
  const int nx = gridDim.x >= 8 ? 8 : 1;
  const int x = (int)(blockIdx.x % nx), slot = (int)(blockIdx.x / nx);
  const int wpx = (int)((gridDim.x - x + nx - 1) / nx);   // workgroups on this XCD
  const int64_t lo = total * x / nx, hi = total * (x + 1) / nx;
  const int my_tiles = lo + slot < hi ? (int)((hi - lo - slot + wpx - 1) / wpx) : 0;
  const int ksteps = (int)((p.K + kPfBK - 1) / kPfBK);
  const int F = my_tiles * ksteps;
  if constexpr (FMT == kNF4) init_pair_table(s_tab, lut);
  if (F == 0) return;

  // Tile descriptors come in through scalar loads (counted by lgkmcnt, so
  // they never disturb the vector-memory counts the stage waits rely on).
  auto meta = [&](int j) {
    PfTile t;
    const int64_t tg = lo + slot + (int64_t)j * wpx;
    const int mt = (int)(tg / n_tiles);
    t.n0 = (int)(tg - (int64_t)mt * n_tiles) * kPfBN;
    t.row0 = t_row0[mt];
    t.rows = t_rows[mt];
    t.e = eids[t_group[mt]];
    return t;
  };

  // ---- per-lane constants
  const int64_t lda2 = p.lda * 2;
  // A stage: wave w fills its kRowsPerWave rows, 8 rows per instruction
  int a_row[kAPieces], a_slot[kAPieces];
#pragma unroll
  for (int i = 0; i < kAPieces; ++i) {
    a_row[i] = wave * kRowsPerWave + i * 8 + (lane >> 3);
    a_slot[i] = (lane & 7) ^ pf_swz(a_row[i] & 15);
  }
  // MFMA k mapping within a 64-wide step: lane half h covers k [32 h, 32 h + 32),
  // MFMA kk (0..3) takes k [32 h + 8 kk, +8) -- 16-byte slot 4 h + kk of a row.
  // Activation operand kk of subtile i: row i * 32 + l32 at i * 4096 + a_off[kk].
  int a_off[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a_off[kk] = l32 * 128 + ((4 * h + kk) ^ pf_swz(l32 & 15)) * 16;

  // ---- ring state
  u32x4_t wreg[kS];      // 16 packed bytes: row n, k [k0 + 32 h, +32)
  unsigned sreg[kS];     // its absmax (NF4) or e8m0 byte (MXFP4)
  PfTile ring_t[kS];
  bool ring_last[kS];
  f32x16_t acc[kMT];
#pragma unroll
  for (int i = 0; i < kMT; ++i) acc[i] = f32x16_t{};

  // ---- issue state: the tile the issue pointer is in. Per tile: buffer
  // resources and per-lane offsets, with rows and columns outside the tile
  // folded into out-of-range offsets; per step only the k offset (a scalar
  // soffset) changes. Steps past the end use zero-size resources, so every
  // step issues the same instructions and the vector-memory counts hold.
  int iss_j = 0, iss_ks = 0;
  PfTile iss_t;
  const char* a_base = nullptr;
  const uint8_t* b_base = nullptr;
  const char* s_base = nullptr;
  int a_bytes = 0, b_bytes = 0, s_bytes = 0;
  int a_voff[kAPieces], b_voff = 0, s_voff = 0;
  auto tile_setup = [&](int j) {
    iss_t = meta(j);
    a_base = reinterpret_cast<const char*>(p.a + (int64_t)iss_t.row0 * p.lda);
    a_bytes = (int)((int64_t)iss_t.rows * lda2);
#pragma unroll
    for (int i = 0; i < kAPieces; ++i)
      a_voff[i] = a_row[i] < iss_t.rows ? (int)(a_row[i] * lda2) + a_slot[i] * 16 : kOOB;
    b_base = p.B + (int64_t)iss_t.e * p.sbe;
    b_bytes = (int)(p.N * p.sbn);
    s_base = static_cast<const char*>(p.S) + (int64_t)iss_t.e * p.sse * kScaleBytes;
    s_bytes = (int)(p.N * p.ssn * kScaleBytes);
    const int64_t n = iss_t.n0 + wave * kWaveCols + l32;
    b_voff = n < p.N ? (int)(n * p.sbn) + h * 16 : kOOB;
    if constexpr (FMT == kNF4) s_voff = n < p.N ? (int)(n * p.ssn * 4) : kOOB;
    else s_voff = n < p.N ? (int)(n * p.ssn) + h : kOOB;
  };
  tile_setup(0);

  auto issue = [&](auto RI, char* stage, bool live) {
    constexpr int r = decltype(RI)::value;
    const int k0 = uniform(iss_ks) * kPfBK;
    live = uniform(live ? 1 : 0) != 0;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a_base), 0, uniform(live ? a_bytes : 0), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(b_base), 0, uniform(live ? b_bytes : 0), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(s_base), 0, uniform(live ? s_bytes : 0), 0x00020000);
#pragma unroll
    for (int i = 0; i < kAPieces; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (lds_ptr_t)(stage + (wave * kAPieces + i) * 1024), 16, a_voff[i], k0 * 2, 0, 0);
    wreg[r] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rb, b_voff, k0 >> 1, 0));
    if constexpr (FMT == kNF4)
      sreg[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, s_voff, (k0 >> 6) * 4, 0);
    else
      sreg[r] = __builtin_amdgcn_raw_buffer_load_b8(rs, s_voff, k0 >> 5, 0);
    ring_t[r] = iss_t;
    ring_last[r] = iss_ks == ksteps - 1;
    // advance
    if (++iss_ks == ksteps) {
      iss_ks = 0;
      ++iss_j;
      if (iss_j < my_tiles) tile_setup(iss_j);
    }
  };

  // Decoded weight operands: wf[r % 2] holds step f's (ring slot r)
  // operands, decoded during step f - 1 (kS is even, so the two buffers
  // alternate without copies).
  u32x4_t wf[2][4];
  auto decode = [&](auto RI) {
    constexpr int r = decltype(RI)::value;
    if constexpr (FMT == kNF4) {
      const float s = __uint_as_float(sreg[r]);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        wf[r & 1][kk] = nf4_dword_to_bf16_at(lds0, wreg[r][kk], lane_off, s);
    } else {
      const float s = e8m0_to_f32(sreg[r]);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) wf[r & 1][kk] = mx_dword_to_bf16(wreg[r][kk], s);
    }
  };

  // MFMAs of step f (slot r) over the first kM activation subtiles. The
  // weights are operand A, so acc[i] holds out^T: lane (l32, h) gets token
  // row i * 32 + l32 and columns 8 g + 4 h + (0..3), g = 0..3.
  auto mma = [&](auto RI, auto MI, const char* stage, auto&& after_first) {
    constexpr int r = decltype(RI)::value;
    constexpr int kM = decltype(MI)::value;
    // operands of k-slices kk and kk + 1 in flight; the reads for kk + 2 go
    // out right after kk's MFMAs, so each MFMA's operand has had a full
    // k-slice of MFMAs to arrive
    u32x4_t av[2][kM];
    auto read = [&](int buf, int kk) {
#pragma unroll
      for (int i = 0; i < kM; ++i)
        av[buf][i] = *reinterpret_cast<const u32x4_t*>(stage + a_off[kk] + i * 4096);
    };
    read(0, 0);
    read(1, 1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kM; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(wf[r & 1][kk]),
                                                          as_bf16x8(av[kk & 1][i]), acc[i], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (kk == 0) {
        after_first();
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kk + 2 < 4) read(kk & 1, kk + 2);
    }
  };

  // The two waves that share a SIMD (w and w + 4) run the step's two halves
  // in opposite orders -- decode of step f + 1 then MFMAs of step f, or the
  // reverse -- so while one wave decodes on the VALU the other keeps the
  // matrix core busy. The order is a template argument of the whole loop
  // (each wave half runs its own copy), so no step merges two orders.
  auto mma_decode = [&](auto RI, auto MI, auto DF, const char* stage, auto&& after_first) {
    constexpr int r = decltype(RI)::value;
    if constexpr (decltype(DF)::value) {
      decode(std::integral_constant<int, (r + 1) % kS>{});
      __builtin_amdgcn_sched_barrier(0);
      mma(RI, MI, stage, after_first);
    } else {
      mma(RI, MI, stage, after_first);
      __builtin_amdgcn_sched_barrier(0);
      decode(std::integral_constant<int, (r + 1) % kS>{});
    }
  };

  auto compute = [&](auto RI, auto DF, const char* stage, auto&& after_first) {
    constexpr int r = decltype(RI)::value;
    const int rows = uniform(ring_t[r].rows);
    // every tile runs all 4 subtiles (rows past the group are zeros in LDS):
    // one straight-line step keeps the accumulators in place
    mma_decode(RI, std::integral_constant<int, 4>{}, DF, stage, after_first);
    if (ring_last[r]) {
      const PfTile t = ring_t[r];
      const int n_l = t.n0 + wave * kWaveCols + 4 * h;   // lane's first column
      uint16_t* o = out + (int64_t)(t.row0 + l32) * p.ldo + n_l;
#pragma unroll
      for (int i = 0; i < kMT; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (i * 32 + l32 < rows && n_l + 8 * g < p.N) {
            uint2 v;
            v.x = bf16x2_bits(acc[i][4 * g + 0], acc[i][4 * g + 1]);
            v.y = bf16x2_bits(acc[i][4 * g + 2], acc[i][4 * g + 3]);
            *reinterpret_cast<uint2*>(o + (int64_t)i * 32 * p.ldo + 8 * g) = v;
          }
        }
        acc[i] = f32x16_t{};
      }
    }
  };

  // Step f: wait for stage f (loads issued after it: the kS - 2 younger
  // stages), barrier, compute; the refill of the stage read in step f - 1
  // with step f + kS - 1 goes out after the first k-slice's MFMAs, so the
  // eight waves' loads do not queue up behind the barrier all at once.
  int f = 0;
  auto step = [&](auto RI, auto DF) {
    constexpr int r = decltype(RI)::value;
    constexpr int rf = (r + kS - 1) % kS;
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<(kS - 2) * kGroupLoads>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const bool live = f + kS - 1 < F;
    compute(RI, DF, stage_of(RI), [&]() {
      issue(std::integral_constant<int, rf>{}, stage_of(std::integral_constant<int, rf>{}), live);
    });
    return ++f < F;
  };

  issue(std::integral_constant<int, 0>{}, s_a0, true);
  issue(std::integral_constant<int, 1>{}, s_a1, F > 1);
  if constexpr (kS > 3) issue(std::integral_constant<int, 2>{}, s_a2, F > 2);
  if constexpr (FMT == kNF4) __syncthreads();  // pair table complete
  decode(std::integral_constant<int, 0>{});
  if (wave < kWaves / 2) {
    auto st = [&](auto RI) { return step(RI, std::true_type{}); };
    while (StepUnroll<0, kS>::run(st)) {
    }
  } else {
    auto st = [&](auto RI) { return step(RI, std::false_type{}); };
    while (StepUnroll<0, kS>::run(st)) {
    }
  }
  // the past-the-end direct-to-LDS loads (zero-size resources) still write
  // their LDS slots: let them land before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt(0);
}

// 256-row tiles (k_prefill_w below).
constexpr int kPtBM = 256;
// cache-policy operand of a buffer store: nt (non-temporal) on gfx950
constexpr int kNonTemporal = 2;
constexpr int kPtStage = kPtBM * kPfBK * 2;

// Pair table with 16 columns: entry (byte b, column c) at b * 128 + c * 8.
__device__ __forceinline__ void init_pair_table16(float2* tab, int lut) {
  const unsigned b = threadIdx.x & 255;
  const float hi = __int_as_float(__builtin_amdgcn_ds_bpermute((int)((b >> 4) << 2), lut));
  const float lo = __int_as_float(__builtin_amdgcn_ds_bpermute((int)((b & 15) << 2), lut));
  const float2 e = make_float2(hi, lo);
  const int j0 = threadIdx.x < 256 ? 0 : 8;
  const int nj = blockDim.x > 256 ? 8 : 16;
  for (int j = 0; j < nj; ++j) tab[b * 16 + ((j0 + j + b) & 15)] = e;
}

// 8 NF4 elements of a dword through the 16-column table: `reg2` holds the
// table address << 1 (bits 8..15 zero) | column * 16.
__device__ __forceinline__ u32x4_t nf4_dword_to_bf16_t16(const char* lds0, unsigned x,
                                                         unsigned reg2, float s) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned addr = __builtin_amdgcn_perm(x, reg2, 0x0C020000u | ((4u + i) << 8)) >> 1;
    const float2 p = *reinterpret_cast<const float2*>(lds0 + addr);
    r[i] = bf16x2_bits(p.x * s, p.y * s);
  }
  return r;
}

// ==================================================== four-wave prefill ==
//
// k_prefill_w<FMT>: the tall-tile forward (256 token rows of one group x 256
// weight rows per tile), 256-thread workgroups, one workgroup per CU and one
// wave per SIMD. Each wave owns 64 weight rows (two 32-row MFMA
// blocks) for all 256 token rows, so
//   * every activation operand read from LDS feeds two MFMAs (half the LDS
//     operand traffic of a 32-row-per-wave split), and
//   * a wave has the whole register file: 256 accumulator registers and room
//     to decode the next step's weights while this step's MFMAs run.
// Everything a step touches comes through LDS rings filled by direct-to-LDS
// loads two steps ahead (activation stages, and per wave the packed weight
// bytes and scales), so the step loop is not unrolled over ring slots and
// the accumulators keep fixed registers.
// The decode of a k-slice is interleaved with the MFMAs of the following
// slice ("rolling" decode): during slice 0 of step f the wave decodes slice 3
// of step f, during slices 1..3 it decodes slices 0..2 of step f + 1, each
// into the operand registers the previous slice's MFMAs released.
// The grid is persistent (by default one workgroup per CU): each XCD
// (workgroup ids go to the XCDs round robin) works through a contiguous
// range of the m-tile-major tile list, its workgroups taking every
// (workgroups per XCD)-th tile of it; the NF4 pair table is built once per
// workgroup.
// The k order of every output element is that of k_prefill, so both give
// identical bits. A tile runs MFMAs and operand reads for its own 32-row
// subtiles only (one instantiation per count, 2..8).
//
// LDS map: activation stages at 0, 32 and 64 KiB; weight ring at 96 KiB
// (three 10 KiB slots: 8 KiB of packed bytes, then the scales); the 16-column
// NF4 pair table at 128 KiB.
constexpr int kPwWaves = 4;
constexpr int kPwRowsPerWave = kPtBM / kPwWaves;           // 64 activation rows staged per wave
constexpr int kPwAPieces = kPtStage / 1024 / kPwWaves;     // 8 direct-to-LDS loads per wave
constexpr int kPwW0 = 3 * kPtStage;                        // weight ring
constexpr int kPwWSlot = 10 * 1024;                     // 8 KiB packed bytes + 4 waves x 2 x 256 B scales
constexpr int kPwTab = 0x20000;                            // 16-column pair table
constexpr int kPwLds = kPwTab + 256 * 16 * 8;              // 160 KiB
static_assert(kPwW0 + 3 * kPwWSlot <= kPwTab, "weight ring below the pair table");

// DG = true: the dgrad form, out[t, k] = sum_n grad[t, n] W[e][n, k]. The
// grad rows stage like the forward's activations (the contraction runs over
// n), t.n0 is the first output column k, and wave w owns the 64 columns
// [t.n0 + 64 w, +64). Its weight operands come from the packed rows read
// transposed: per step the wave's slot holds 64 rows (n) x 32 bytes (its 64
// k), and one ds_read_b64_tr_b8 per slice hands each lane one byte column c
// of the slice's 8 rows (lane half h: rows 32 h + 8 kk + 0..7, as the
// forward's k mapping). Byte c holds k = 2c (high nibble) and 2c + 1 (low
// nibble), which feed the two 32-column MFMA blocks b = 0 (even k) and
// b = 1 (odd k), so block b, MFMA row i is column t.n0 + 64 w + 2 i + b.
// The 16-byte rows of the tr8 read come in the order 0,2,4,6,1,3,5,7, so
// dword 0 of the result holds the even rows and dword 1 the odd ones, and
// the bf16 pairs (row 2m, row 2m + 1) come out of byte m of each. The
// absmax of (row, the wave's 64-block) is staged per step as 64 floats.
// MXFP4 (low nibble = even k) converts each row's byte with that row's e8m0
// scale of the lane's 32-column block and pairs rows with a byte permute.
template <int FMT, int kM, bool DG>
__device__ __forceinline__ void prefill_w_tile(const FwdArgs& p, const PfTile t, char* smem,
                                               uint16_t* __restrict__ out, const int lut,
                                               const bool build_table) {
  const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  constexpr int kScaleBytes = FMT == kNF4 ? 4 : 1;
  // contraction length (forward: K; dgrad: N) and output width (N; K)
  const int64_t Kc = DG ? p.N : p.K;
  const int64_t Nout = DG ? p.K : p.N;
  const int F = (int)((Kc + kPfBK - 1) / kPfBK);
  // per step: activation pieces, 2 weight-byte loads, scale loads (NF4: one
  // of 64 rows; MXFP4: two of 32 rows x 2 blocks)
  constexpr int kGroupLoads = kPwAPieces + 2 + (FMT == kNF4 ? 1 : 2);
  // table address << 1 | column * 16 (nf4_dword_to_bf16_t16)
  const unsigned reg2 = ((unsigned)kPwTab << 1) | (unsigned)(lane & 15) * 16u;

  // k mapping within a 64-wide step (as in k_prefill): lane half h covers
  // k [32 h, 32 h + 32); MFMA slice kk takes k [32 h + 8 kk, +8).
  int a_off[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a_off[kk] = l32 * 128 + ((4 * h + kk) ^ pf_swz(l32 & 15)) * 16;

  // ---- per-tile load descriptors: rows and columns outside the tile fold
  // into out-of-range offsets; per step only the k offset (soffset) moves
  const char* a_base = reinterpret_cast<const char*>(p.a + (int64_t)t.row0 * p.lda);
  const int a_bytes = (int)((int64_t)t.rows * p.lda * 2);
  int a_voff[kPwAPieces];
#pragma unroll
  for (int i = 0; i < kPwAPieces; ++i) {
    // staged row wave * 64 + 8 i + lane / 8, 16-byte slot (lane % 8) ^ swizzle
    const int row = wave * kPwRowsPerWave + i * 8 + (lane >> 3);
    const int slot16 = (lane & 7) ^ pf_swz(row & 15);
    a_voff[i] = row < t.rows ? (int)(row * p.lda * 2) + slot16 * 16 : kOOB;
  }
  const uint8_t* b_base = p.B + (int64_t)t.e * p.sbe;
  const char* s_base = static_cast<const char*>(p.S) + (int64_t)t.e * p.sse * kScaleBytes;
  const int b_bytes = (int)(p.N * p.sbn);
  const int s_bytes = (int)(p.N * p.ssn * kScaleBytes);
  int b_voff[2], s_voff[2];
  if constexpr (DG) {
    // step rows n0 + 32 rb + lane / 2, 16 bytes (lane % 2) of the wave's 32;
    // per step only soffset (n0 rows) moves. A wave past K loads zeros.
    const int64_t kw = t.n0 + wave * 64;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
      b_voff[rb] = kw < p.K ? (int)((rb * 32 + (lane >> 1)) * p.sbn + kw / 2) + (lane & 1) * 16 : kOOB;
    if constexpr (FMT == kNF4) {
      s_voff[0] = kw < p.K ? (int)(lane * p.ssn * 4 + (kw >> 6) * 4) : kOOB;
      s_voff[1] = kOOB;
    } else {
      // two e8m0 blocks (32 k each) per row: load bl stages block bl of 64 rows
#pragma unroll
      for (int bl = 0; bl < 2; ++bl)
        s_voff[bl] = kw < p.K ? (int)(lane * p.ssn + (kw >> 5) + bl) : kOOB;
    }
  } else {
    // loading lane i: row 32 rb + i / 2 of the wave's 64, 16-byte half i % 2
    // (two lanes per row keep each lane quad on two cache lines); NF4
    // scales: row i, one load; MXFP4 scales: row 32 rb + i / 2, block i % 2
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int64_t n = t.n0 + wave * 64 + rb * 32 + (lane >> 1);
      b_voff[rb] = n < p.N ? (int)(n * p.sbn) + (lane & 1) * 16 : kOOB;
      if constexpr (FMT != kNF4) s_voff[rb] = n < p.N ? (int)(n * p.ssn) + (lane & 1) : kOOB;
    }
    if constexpr (FMT == kNF4) {
      const int64_t n = t.n0 + wave * 64 + lane;
      s_voff[0] = n < p.N ? (int)(n * p.ssn * 4) : kOOB;
      s_voff[1] = kOOB;
    }
  }
  // this wave's blocks of a weight slot: bytes (rb) at +rb KiB, lane-linear;
  // scales one dword per lane (direct-to-LDS loads of a byte still land in
  // a dword slot per lane)
  const int w_wave = (wave * 2) * 1024;
  const int s_wave = 8192 + (wave * 2) * 256;

  // issue step g's loads: activation stage g % 3, weight slot g % 3 (zero-size
  // resources past the end, so every step issues the same loads and the
  // vector-memory counts hold)
  // Loads are issued in parts (so a slice never issues more than a few):
  // activation pieces [p0, p1) of step g, and weight loads [q0, q1) of step g
  // (0, 1: packed bytes of row blocks 0, 1; 2, 3: their scales).
  auto issue_a = [&](int g, int p0, int p1) {
    const bool live = g < F;
    const int k0 = live ? g * kPfBK : 0;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a_base), 0, uniform(live ? a_bytes : 0), 0x00020000);
    char* stage = smem + uniform((g % 3) * kPtStage) + wave * kPwAPieces * 1024;
#pragma unroll
    for (int i = 0; i < kPwAPieces; ++i)
      if (i >= p0 && i < p1)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(stage + i * 1024), 16, a_voff[i],
                                                 uniform(k0 * 2), 0, 0);
  };
  auto issue_w = [&](int g, int q0, int q1) {
    const bool live = g < F;
    const int k0 = live ? g * kPfBK : 0;
    if constexpr (DG) {
      // rows [k0, k0 + 64) of the contraction: 2 KiB of bytes, 64 scales
      const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
          uniform_ptr(b_base), 0, uniform(live ? b_bytes : 0), 0x00020000);
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          uniform_ptr(s_base), 0, uniform(live ? s_bytes : 0), 0x00020000);
      char* slot = smem + kPwW0 + uniform((g % 3) * kPwWSlot);
#pragma unroll
      for (int b = 0; b < 2; ++b)
        if (b >= q0 && b < q1)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(slot + w_wave + b * 1024), 16,
                                                   b_voff[b], uniform((int)(k0 * p.sbn)), 0, 0);
      if constexpr (FMT == kNF4) {
        if (2 >= q0 && 2 < q1)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(slot + s_wave), 4, s_voff[0],
                                                   uniform((int)(k0 * p.ssn * 4)), 0, 0);
      } else {
#pragma unroll
        for (int bl = 0; bl < 2; ++bl)
          if (bl + 2 >= q0 && bl + 2 < q1)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(slot + s_wave + bl * 256), 1,
                                                     s_voff[bl], uniform((int)(k0 * p.ssn)), 0, 0);
      }
      return;
    }
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(b_base), 0, uniform(live ? b_bytes : 0), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(s_base), 0, uniform(live ? s_bytes : 0), 0x00020000);
    char* slot = smem + kPwW0 + uniform((g % 3) * kPwWSlot);
#pragma unroll
    for (int b = 0; b < 2; ++b)
      if (b >= q0 && b < q1)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(slot + w_wave + b * 1024), 16,
                                                 b_voff[b], uniform(k0 >> 1), 0, 0);
    if constexpr (FMT == kNF4) {
      if (2 >= q0 && 2 < q1)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(slot + s_wave), 4, s_voff[0],
                                                 uniform((k0 >> 6) * 4), 0, 0);
    } else {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        if (b + 2 < q0 || b + 2 >= q1) continue;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(slot + s_wave + b * 256), 1,
                                                 s_voff[b], uniform(k0 >> 5), 0, 0);
      }
    }
  };
  // this lane's packed bytes and scale of step g (block rb), from its slot
  // dgrad: lane address of the tr8 read of slice kk (lane i of its 16-lane
  // group supplies 8 bytes of row pi(i / 2), half i % 2 of the group's 16)
  const int tr_off = w_wave + (32 * h + ((lane >> 1) & 3) * 2 + ((lane >> 3) & 1)) * 32 +
                     ((lane >> 4) & 1) * 16 + (lane & 1) * 8;
  auto read_w = [&](int g, u32x4_t (&w)[2], float (&sc)[2]) {
    const char* slot = smem + kPwW0 + uniform((g % 3) * kPwWSlot);
    if constexpr (DG) {
      typedef __attribute__((address_space(3))) v2i32_t lds_v2i32;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const v2i32_t r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i32*)(lds_ptr_t)(slot + tr_off + kk * 8 * 32));
        w[0][kk] = (unsigned)r.x;
        w[1][kk] = (unsigned)r.y;
      }
      sc[0] = sc[1] = 0.f;
      return;
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      w[b] = *reinterpret_cast<const u32x4_t*>(slot + w_wave + b * 1024 + (2 * l32 + h) * 16);
      if constexpr (FMT == kNF4)
        sc[b] = *reinterpret_cast<const float*>(slot + s_wave + (b * 32 + l32) * 4);
      else
        sc[b] = e8m0_to_f32(
            *reinterpret_cast<const uint8_t*>(slot + s_wave + b * 256 + (2 * l32 + h) * 4));
    }
  };

  // wf[rb][kk]: the weight operand of slice kk (rows of block rb).
  u32x4_t wf[2][4];
  // Two-phase decode of one slice of weights (a "target"): the lookup phase
  // (NF4 pair-table reads) runs one slice ahead of the math phase (scale
  // multiply, bf16 pack), so the table reads' latency hides behind a slice of
  // MFMAs. Parity q alternates between targets.
  float2 tp[2][2][4];   // NF4: table pairs [q][rb][byte of the dword]
  unsigned traw[2][2];  // MXFP4: the packed dword [q][rb]
  float ts[2][2];       // the target's scale [q][rb]
  float ts8[2][DG ? 8 : 1];   // dgrad: the scales of the target's 8 rows [q][row]
  // Both phases come in 8 pieces (pc), so the slice loop can spread them
  // over its MFMA pairs.
  // Lookup piece pc: NF4 table pair of byte pc % 4 of dword pc / 4 (dgrad:
  // piece 0 also reads the target rows' 8 scales); MXFP4 keeps dword pc.
  // (dgrad) g, kk: the target's step and slice, whose rows' scales it reads
  auto lookup_pc = [&](auto QI, unsigned x0, unsigned x1, const float (&sc)[2], int g, int kk,
                       int pc) {
    constexpr int q = decltype(QI)::value;
    const int b = pc >> 2, i = pc & 3;
    const unsigned xb = b ? x1 : x0;
    if constexpr (DG) {
      if (pc == 0) {
        // MXFP4: the lane's byte column c = lane % 32 holds k = 2c, 2c + 1,
        // in scale block c / 16; each staged byte sits in its own dword
        const char* sp = smem + kPwW0 + uniform((g % 3) * kPwWSlot) + s_wave + (32 * h + 8 * kk) * 4 +
                         (FMT == kNF4 ? 0 : (l32 >> 4) * 256);
        const u32x4_t s0 = *reinterpret_cast<const u32x4_t*>(sp);
        const u32x4_t s1 = *reinterpret_cast<const u32x4_t*>(sp + 16);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (FMT == kNF4) {
            ts8[q][r] = __uint_as_float(s0[r]);
            ts8[q][4 + r] = __uint_as_float(s1[r]);
          } else {
            ts8[q][r] = e8m0_to_f32(s0[r] & 0xFFu);
            ts8[q][4 + r] = e8m0_to_f32(s1[r] & 0xFFu);
          }
        }
      }
      if constexpr (FMT != kNF4) {
        if (pc < 2) traw[q][pc] = pc ? x1 : x0;
        return;
      }
    }
    if constexpr (FMT == kNF4) {
      if (i == 0) ts[q][b] = sc[b];
      unsigned addr = __builtin_amdgcn_perm(xb, reg2, 0x0C020000u | ((4u + i) << 8)) >> 1;
      tp[q][b][i] = *reinterpret_cast<const float2*>(smem + addr);
    } else {
      if (pc < 2) {
        traw[q][pc] = pc ? x1 : x0;
        ts[q][pc] = sc[pc];
      }
    }
  };
  // Math piece pc: one bf16-pair dword of operand block pc / 4, dword pc % 4
  // (dgrad: dword pc / 2 of block pc % 2); MXFP4 converts block pc whole.
  auto math_pc = [&](auto QI, auto DI, int pc) {
    constexpr int q = decltype(QI)::value;
    constexpr int d = decltype(DI)::value;
    if constexpr (DG && FMT != kNF4) {
      // byte m of dword 0 / 1: rows 2m / 2m + 1, low nibble even k; the
      // convert applies each row's own scale, a byte permute pairs the rows
      if (pc & 1) return;
      const int m = pc >> 1;
      auto cvt = [&](unsigned x, float sc) {
        bf16x2_t v;
        if (m == 0) v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 0);
        else if (m == 1) v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 1);
        else if (m == 2) v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 2);
        else v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, sc, 3);
        return __builtin_bit_cast(unsigned, v);
      };
      const unsigned c0 = cvt(traw[q][0], ts8[q][2 * m]);
      const unsigned c1 = cvt(traw[q][1], ts8[q][2 * m + 1]);
      wf[0][d][m] = __builtin_amdgcn_perm(c1, c0, 0x05040100u);
      wf[1][d][m] = __builtin_amdgcn_perm(c1, c0, 0x07060302u);
    } else if constexpr (DG) {
      // byte m of dword 0 / 1: rows 2m / 2m + 1; .x even k, .y odd k
      const int m = pc >> 1;
      if (pc & 1)
        wf[1][d][m] = bf16x2_bits(tp[q][0][m].y * ts8[q][2 * m], tp[q][1][m].y * ts8[q][2 * m + 1]);
      else
        wf[0][d][m] = bf16x2_bits(tp[q][0][m].x * ts8[q][2 * m], tp[q][1][m].x * ts8[q][2 * m + 1]);
    } else if constexpr (FMT == kNF4) {
      const int b = pc >> 2, i = pc & 3;
      wf[b][d][i] = bf16x2_bits(tp[q][b][i].x * ts[q][b], tp[q][b][i].y * ts[q][b]);
    } else {
      if (pc < 2) wf[pc][d] = mx_dword_to_bf16(traw[q][pc], ts[q][pc]);
    }
  };
  auto lookup = [&](auto QI, unsigned x0, unsigned x1, const float (&sc)[2], int g, int kk) {
#pragma unroll
    for (int pc = 0; pc < 8; ++pc) lookup_pc(QI, x0, x1, sc, g, kk, pc);
  };
  auto math = [&](auto QI, auto DI) {
#pragma unroll
    for (int pc = 0; pc < 8; ++pc) math_pc(QI, DI, pc);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  // ---- pipeline. The loads of group g (activation stage of step g + 2,
  // weights of step g + 3) start in slice 3 of step g - 1, right after the
  // barrier that publishes step g's stage, and are spread over the next four
  // slices (three per slice), so the barrier, the load issue and the operand
  // reads of the next step's slice 0 all overlap MFMAs.
  auto ao_of = [&](int g, int kk) { return a_off[kk] + uniform((g % 3) * kPtStage); };

  // prologue: weights of step 0, groups -2 and -1
  issue_w(0, 0, 4);
  issue_a(0, 0, 8);
  // the NF4 pair table is built while the first loads are in flight
  if constexpr (FMT == kNF4)
    if (build_table) init_pair_table16(reinterpret_cast<float2*>(smem + kPwTab), lut);
  // step 0's weight bytes and scales have landed (the activation pieces may
  // not have): their cache lines also hold the next steps' bytes and scales
  // of the same rows, so steps 1 and 2 hit in L2 instead of queueing a second
  // and third miss per row behind the first
  wait_vm_lgkm0<kPwAPieces>();
  issue_w(1, 0, 4);
  issue_a(1, 0, 8);
  issue_w(2, 0, 4);
  // step 0's stage and step 1's weights have landed for every wave, the
  // pair table is complete
  wait_vm_lgkm0<kGroupLoads>();
  __builtin_amdgcn_s_barrier();
  issue_a(2, 0, 3);   // the rest of this group goes out during step 0
  u32x4_t wn[2];
  float sn[2];
  read_w(0, wn, sn);
  lookup(I1{}, wn[0][0], wn[1][0], sn, 0, 0);
  math(I1{}, I0{});
  lookup(I1{}, wn[0][1], wn[1][1], sn, 0, 1);
  math(I1{}, I1{});
  lookup(I1{}, wn[0][2], wn[1][2], sn, 0, 2);
  math(I1{}, I2{});
  lookup(I0{}, wn[0][3], wn[1][3], sn, 0, 3);   // step 0's slice 3, decoded during its slice 0
  read_w(1, wn, sn);
  u32x4_t av[kM];
#pragma unroll
  for (int i = 0; i < kM; ++i)
    av[i] = *reinterpret_cast<const u32x4_t*>(smem + ao_of(0, 0) + i * 4096);
  f32x16_t acc[2][kM];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < kM; ++i) acc[b][i] = f32x16_t{};

  // instruction mix of one slice, for the interleaving below

  for (int f = 0; f < F; ++f) {
    int ao[4];
#pragma unroll
    for (int kk = 1; kk < 4; ++kk) ao[kk] = ao_of(f, kk);
    ao[0] = ao_of(f + 1, 0);
    // slice kk: its MFMAs, the next slice's operand reads, the lookup of the
    // next target and the math of this slice's target (target of slice 0:
    // this step's slice 3; of slices 1..3: the next step's slices 0..2).
    // wn holds step f + 1's packed bytes.
    auto slice = [&](auto KI) {
      constexpr int kk = decltype(KI)::value;
      __builtin_amdgcn_sched_barrier(0);
      // this slice's lookup input: for slice 3 it is saved before step
      // f + 2's bytes replace wn
      unsigned x0 = wn[0][kk], x1 = wn[1][kk];
      float xs[2] = {sn[0], sn[1]};
      if constexpr (kk == 3) {
        // step f + 1's stage and step f + 2's weights have landed, every
        // wave has read all of stage f: publish, and start refilling it
        wait_vm_lgkm0<kGroupLoads>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        read_w(f + 2, wn, sn);
      }
      constexpr int qn = (kk + 1) & 1, qc = kk & 1;
      using QN = std::integral_constant<int, qn>;
      using QC = std::integral_constant<int, qc>;
      using DT = std::integral_constant<int, (kk + 3) & 3>;
      // per 32-row subtile i: its two MFMAs, the reload of its operand for
      // the next slice, and its share (pieces 8 i / kM .. 8 (i + 1) / kM) of
      // the lookup (next target) and of the math (this slice's target),
      // fenced so that the decode work sits between MFMAs and runs while
      // they execute
#pragma unroll
      for (int i = 0; i < kM; ++i) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[b][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              as_bf16x8(wf[b][kk]), as_bf16x8(av[i]), acc[b][i], 0, 0, 0);
        av[i] = *reinterpret_cast<const u32x4_t*>(smem + ao[(kk + 1) & 3] + i * 4096);
        // this slice's share of the loads of group f + 1 (stage of step
        // f + 3, weights of step f + 4; started in slice 3 of step f): three
        // loads, spread over the subtiles so the vector-memory queue never
        // takes a burst
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          if ((j * kM) / 3 != i) continue;
          if constexpr (kk == 0) issue_a(f + 2, 3 + j, 4 + j);
          if constexpr (kk == 1) {
            if (j < 2) issue_a(f + 2, 6 + j, 7 + j);
            else issue_w(f + 3, 0, 1);
          }
          if constexpr (kk == 2) issue_w(f + 3, 1 + j, 2 + j);
          if constexpr (kk == 3) issue_a(f + 3, j, j + 1);
        }
#pragma unroll
        for (int pc = (8 * i) / kM; pc < (8 * (i + 1)) / kM; ++pc) {
          lookup_pc(QN{}, x0, x1, xs, f + 1, kk, pc);
          math_pc(QC{}, DT{}, pc);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    slice(I0{});
    slice(I1{});
    slice(I2{});
    slice(I3{});
  }

  // ---- epilogue: the bf16 tile goes through LDS (free now: every wave is
  // past its last operand read), so the global stores write whole rows.
  // LDS tile: row r at r * 512 bytes, 16-byte chunk c at (c ^ (r % 32)) * 16.
  // Every load must have landed first, the past-the-end ones included: a
  // direct-to-LDS load through a zero-size resource still writes (zeros) to
  // its LDS slot, which the tile below overlaps.
  __builtin_amdgcn_sched_barrier(0);
  wait_vm_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  if constexpr (DG) {
    // MFMA row 8 g + 4 h + q of block b is column 64 w + 2 (8 g + 4 h + q) + b:
    // the two blocks interleave into one 16-byte chunk 8 w + 2 g + h
#pragma unroll
    for (int i = 0; i < kM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = i * 32 + l32;
        const int chunk = wave * 8 + 2 * g + h;
        u32x4_t v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = bf16x2_bits(acc[0][i][4 * g + q], acc[1][i][4 * g + q]);
        *reinterpret_cast<u32x4_t*>(smem + row * 512 + ((chunk ^ l32) << 4)) = v;
      }
  } else
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < kM; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = i * 32 + l32;
        const int col = wave * 64 + b * 32 + 8 * g + 4 * h;   // 4 columns
        u32x2_t v;
        v.x = bf16x2_bits(acc[b][i][4 * g + 0], acc[b][i][4 * g + 1]);
        v.y = bf16x2_bits(acc[b][i][4 * g + 2], acc[b][i][4 * g + 3]);
        *reinterpret_cast<u32x2_t*>(smem + row * 512 + (((col >> 3) ^ l32) << 4) + (col & 7) * 2) = v;
      }
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(out + (int64_t)t.row0 * p.ldo), 0, uniform((int)((int64_t)t.rows * p.ldo * 2)),
      0x00020000);
  const int ldo2 = (int)(p.ldo * 2);
  // whole 8-column chunks store 16 bytes; the chunk that straddles the
  // output width (width % 8 == 4) stores its first 8 bytes only, so no
  // store reaches past a row's last column. The stores are non-temporal
  // (nt): the output is not read again here, and every CU reaches its
  // epilogue at about the same time, so a tile's 128 KiB would otherwise
  // push the next tiles' weights and activations out of L2 (down
  // projection at M = 256: 760 -> 813 TFLOP/s).
  const int chunk = lane & 31;
  const int col = t.n0 + chunk * 8;
  const int coff16 = col + 8 <= Nout ? col * 2 + h * ldo2 : kOOB;
  const int coff8 = col < Nout && col + 8 > Nout ? col * 2 + h * ldo2 : kOOB;
  const bool straddle = Nout % 8 != 0;
  // wave w stores rows 2 (4 j + w) + lane / 32, j = 0 .. 4 kM - 1
#pragma unroll
  for (int j = 0; j < kM * 4; ++j) {
    const int row = (j * 4 + wave) * 2 + h;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(smem + row * 512 + ((chunk ^ (row & 31)) << 4));
    const int so = uniform((j * 4 + wave) * 2 * ldo2);
    __builtin_amdgcn_raw_buffer_store_b128(v, ro, coff16, so, kNonTemporal);
    if (straddle) {
      u32x2_t v2;
      v2.x = v[0];
      v2.y = v[1];
      __builtin_amdgcn_raw_buffer_store_b64(v2, ro, coff8, so, kNonTemporal);
    }
  }
}

// A tile table small enough to travel in the kernel arguments (n > 0): no
// upload, so a call needs no copy ahead of its launch (and a captured graph
// no copy node). grp holds the group index, or the expert id itself where
// the caller knows the ids on the host (grp_is_expert). 3 KiB, inside the
// kernel-argument limit with FwdArgs.
constexpr int kPwMaxTiles = 256;
struct PwTiles {
  int32_t row0[kPwMaxTiles];
  int32_t rows[kPwMaxTiles];
  int32_t grp[kPwMaxTiles];
  int32_t n;
  int32_t grp_is_expert;
};

template <int FMT, bool DG = false>
__global__ void __launch_bounds__(256, 1)
    k_prefill_w(const FwdArgs p, const int32_t* __restrict__ t_row0,
                const int32_t* __restrict__ t_rows, const int32_t* __restrict__ t_group,
                const int32_t* __restrict__ eids, uint16_t* __restrict__ out, const PwTiles tt) {
  __shared__ __attribute__((aligned(16))) char smem[kPwLds];
  const int lut = FMT == kNF4 ? nf4_lut_lane() : 0;
  __builtin_amdgcn_sched_barrier(0);

  // XCD x = blockIdx % 8 takes the x-th contiguous eighth of the tile list;
  // its workgroups walk that range with a stride of their count (tiles come
  // largest first, so each workgroup gets one tile of every size band)
  const int n_tiles = (int)(((DG ? p.K : p.N) + kPfBN - 1) / kPfBN);
  const int64_t total = (int64_t)p.n_mtiles * n_tiles;
  const int nx = gridDim.x >= 8 ? 8 : 1;
  const int x = (int)(blockIdx.x % nx), idx = (int)(blockIdx.x / nx);
  const int stride = (int)(gridDim.x / nx);
  const int64_t lo = total * x / nx, hi = total * (x + 1) / nx;
  bool first = true;
  for (int64_t tg = lo + idx; tg < hi; tg += stride) {
    if (!first) {
      // every wave is past the previous tile's epilogue reads of the LDS
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
    }
    PfTile t;
    const int mt = (int)(tg / n_tiles);
    t.n0 = (int)(tg - (int64_t)mt * n_tiles) * kPfBN;
    if (tt.n > 0) {
      // the table in the kernel arguments (scalar loads from the kernarg
      // segment)
      t.row0 = tt.row0[mt];
      t.rows = tt.rows[mt];
      t.e = tt.grp_is_expert ? tt.grp[mt] : eids[tt.grp[mt]];
    } else {
      t.row0 = t_row0[mt];
      t.rows = t_rows[mt];
      t.e = eids[t_group[mt]];
    }
    // MFMAs for the tile's 32-row subtiles only
    switch ((t.rows + 31) >> 5) {
      case 8: prefill_w_tile<FMT, 8, DG>(p, t, smem, out, lut, first); break;
      case 7: prefill_w_tile<FMT, 7, DG>(p, t, smem, out, lut, first); break;
      case 6: prefill_w_tile<FMT, 6, DG>(p, t, smem, out, lut, first); break;
      case 5: prefill_w_tile<FMT, 5, DG>(p, t, smem, out, lut, first); break;
      case 4: prefill_w_tile<FMT, 4, DG>(p, t, smem, out, lut, first); break;
      case 3: prefill_w_tile<FMT, 3, DG>(p, t, smem, out, lut, first); break;
      default: prefill_w_tile<FMT, 2, DG>(p, t, smem, out, lut, first); break;
    }
    first = false;
  }
}

// ========================================================== tiled dgrad ==
//
// out[t, k] = sum_n grad[t, n] W[e][n, k]: the weights are read transposed.
// Same skeleton as k_prefill -- 128-row tiles of one group x 256 output
// columns (here: k), a persistent XCD-contiguous tile list, a 4-stage ring of
// gradient rows filled by direct-to-LDS loads, one flat pipeline over (tile,
// 64-wide n-step) -- with the weight operand going through LDS:
//   * per step each thread loads 4 packed rows (n) x 8 columns (k) -- one
//     dword per row -- decodes them and writes them transposed (k-major, 4
//     consecutive n per 8-byte write) into a double-buffered bf16 tile of 256
//     k-rows x 64 n, decoded during the step before the one that reads it;
//   * wave w reads its 32 k-rows of that tile as MFMA operand A and the
//     gradient rows from the stage as operand B (32 x 32 x 16 bf16).
// The NF4 pair table here has 16 lane columns (32 KiB), so stages, weight
// tiles and table fit the 160 KiB of LDS.
constexpr int kDgTile = kPfBN;            // output columns (k) per tile
constexpr int kDgStep = 64;               // n per step
constexpr int kDgBStage = kDgTile * kDgStep * 2;

template <int FMT>
__global__ void __launch_bounds__(512, 2)
    k_dgrad_tiled(const FwdArgs p, const int32_t* __restrict__ t_row0,
                  const int32_t* __restrict__ t_rows, const int32_t* __restrict__ t_group,
                  const int32_t* __restrict__ eids, uint16_t* __restrict__ out) {
  constexpr int kS = 4;
  constexpr int kWaves = 8;
  constexpr int kAPieces = kPfStage / 1024 / kWaves;
  constexpr int kRowsPerWave = kPfBM / kWaves;
  constexpr int kGroupLoads = kAPieces + 5;          // + 4 weight dwords + 1 scale
  constexpr int kMT = kPfBM / 32;
  constexpr int kScaleBytes = FMT == kNF4 ? 4 : 1;
  __shared__ __attribute__((aligned(16))) char s_a0[kPfStage];
  __shared__ __attribute__((aligned(16))) char s_a1[kPfStage];
  __shared__ __attribute__((aligned(16))) char s_a2[kPfStage];
  __shared__ __attribute__((aligned(16))) char s_a3[kPfStage];
  __shared__ __attribute__((aligned(16))) char s_b0[kDgBStage];
  __shared__ __attribute__((aligned(16))) char s_b1[kDgBStage];
  extern __shared__ __attribute__((aligned(16))) float2 s_tab[];   // NF4: 32 KiB at 0x20000
  auto stage_of = [&](auto RI) -> char* {
    constexpr int r = decltype(RI)::value;
    if constexpr (r == 0) return s_a0;
    else if constexpr (r == 1) return s_a1;
    else if constexpr (r == 2) return s_a2;
    else return s_a3;
  };
  auto bbuf_of = [&](auto RI) -> char* {
    if constexpr ((decltype(RI)::value & 1) == 0) return s_b0;
    else return s_b1;
  };
  const int lut = FMT == kNF4 ? nf4_lut_lane() : 0;
  __builtin_amdgcn_sched_barrier(0);
  const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  // decode role: rows 4 rg .. 4 rg + 3 of the step, columns 8 kc .. 8 kc + 7
  const int rg = lane & 15, kc = wave * 4 + (lane >> 4);
  const unsigned tab_base = (unsigned)(uintptr_t)s_tab;
  const unsigned reg2 = (tab_base << 1) | (unsigned)(lane & 15) * 16u;
  const char* lds0 = reinterpret_cast<const char*>(s_tab) - tab_base;

  // ---- tiles (output columns k in tiles of 256)
  const int n_tiles = (int)((p.K + kDgTile - 1) / kDgTile);
  const int64_t total = (int64_t)p.n_mtiles * n_tiles;
  const int nx = gridDim.x >= 8 ? 8 : 1;
  const int x = (int)(blockIdx.x % nx), slot = (int)(blockIdx.x / nx);
  const int wpx = (int)((gridDim.x - x + nx - 1) / nx);
  const int64_t lo = total * x / nx, hi = total * (x + 1) / nx;
  const int my_tiles = lo + slot < hi ? (int)((hi - lo - slot + wpx - 1) / wpx) : 0;
  const int ksteps = (int)(p.N / kDgStep);
  const int F = my_tiles * ksteps;
  if constexpr (FMT == kNF4) init_pair_table16(s_tab, lut);
  if (F == 0) return;

  auto meta = [&](int j) {
    PfTile t;
    const int64_t tg = lo + slot + (int64_t)j * wpx;
    const int mt = (int)(tg / n_tiles);
    t.n0 = (int)(tg - (int64_t)mt * n_tiles) * kDgTile;   // first output column
    t.row0 = t_row0[mt];
    t.rows = t_rows[mt];
    t.e = eids[t_group[mt]];
    return t;
  };

  const int64_t lda2 = p.lda * 2;
  int a_row[kAPieces], a_slot[kAPieces];
#pragma unroll
  for (int i = 0; i < kAPieces; ++i) {
    a_row[i] = wave * kRowsPerWave + i * 8 + (lane >> 3);
    a_slot[i] = (lane & 7) ^ pf_swz(a_row[i] & 15);
  }
  // MFMA kk (0..3) contracts n [16 kk + 8 h, +8): 16-byte slot 2 kk + h of a
  // row in both the gradient stage and the weight tile.
  int a_off[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a_off[kk] = l32 * 128 + ((2 * kk + h) ^ pf_swz(l32 & 15)) * 16;
  const int b_wave = wave * 32 * 128;

  unsigned wreg[kS][4];
  // scale of row n0 + lane of the wave's 32 columns (one scale block: the
  // columns are 32-aligned); threads pick their rows' with ds_bpermute
  unsigned sreg[kS];
  PfTile ring_t[kS];
  bool ring_last[kS];
  f32x16_t acc[kMT];
#pragma unroll
  for (int i = 0; i < kMT; ++i) acc[i] = f32x16_t{};

  int iss_j = 0, iss_ks = 0;
  PfTile iss_t;
  const char* a_base = nullptr;
  const uint8_t* b_base = nullptr;
  const char* s_base = nullptr;
  int a_bytes = 0, b_bytes = 0, s_bytes = 0;
  int a_voff[kAPieces], b_voff[4], s_voff = 0;
  auto tile_setup = [&](int j) {
    iss_t = meta(j);
    a_base = reinterpret_cast<const char*>(p.a + (int64_t)iss_t.row0 * p.lda);
    a_bytes = (int)((int64_t)iss_t.rows * lda2);
#pragma unroll
    for (int i = 0; i < kAPieces; ++i)
      a_voff[i] = a_row[i] < iss_t.rows ? (int)(a_row[i] * lda2) + a_slot[i] * 16 : kOOB;
    b_base = p.B + (int64_t)iss_t.e * p.sbe;
    b_bytes = (int)(p.N * p.sbn);
    s_base = static_cast<const char*>(p.S) + (int64_t)iss_t.e * p.sse * kScaleBytes;
    s_bytes = (int)(p.N * p.ssn * kScaleBytes);
    const int64_t c = iss_t.n0 + kc * 8;                 // first output column of the thread
    const bool ok = c < p.K;
#pragma unroll
    for (int i = 0; i < 4; ++i) b_voff[i] = ok ? (int)((4 * rg + i) * p.sbn + (c >> 1)) : kOOB;
    const int64_t cw = iss_t.n0 + wave * 32;             // the wave's first column
    if constexpr (FMT == kNF4) s_voff = cw < p.K ? (int)((lane * p.ssn + (cw >> 6)) * 4) : kOOB;
    else s_voff = cw < p.K ? (int)(lane * p.ssn + (cw >> 5)) : kOOB;
  };
  tile_setup(0);

  auto issue = [&](auto RI, char* stage, bool live) {
    constexpr int r = decltype(RI)::value;
    const int n0 = uniform(iss_ks) * kDgStep;
    live = uniform(live ? 1 : 0) != 0;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(a_base), 0, uniform(live ? a_bytes : 0), 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(b_base), 0, uniform(live ? b_bytes : 0), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(s_base), 0, uniform(live ? s_bytes : 0), 0x00020000);
#pragma unroll
    for (int i = 0; i < kAPieces; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (lds_ptr_t)(stage + (wave * kAPieces + i) * 1024), 16, a_voff[i], n0 * 2, 0, 0);
    const int b_soff = uniform((int)(n0 * p.sbn));
    const int s_soff = uniform((int)(n0 * p.ssn * kScaleBytes));
#pragma unroll
    for (int i = 0; i < 4; ++i) wreg[r][i] = __builtin_amdgcn_raw_buffer_load_b32(rb, b_voff[i], b_soff, 0);
    if constexpr (FMT == kNF4) sreg[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, s_voff, s_soff, 0);
    else sreg[r] = __builtin_amdgcn_raw_buffer_load_b8(rs, s_voff, s_soff, 0);
    ring_t[r] = iss_t;
    ring_last[r] = iss_ks == ksteps - 1;
    if (++iss_ks == ksteps) {
      iss_ks = 0;
      ++iss_j;
      if (iss_j < my_tiles) tile_setup(iss_j);
    }
  };

  // Decode the weights of ring slot r into weight tile r & 1 (transposed).
  auto decode = [&](auto RI) {
    constexpr int r = decltype(RI)::value;
    char* bb = bbuf_of(RI);
    u32x4_t rowv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const unsigned sc = (unsigned)__builtin_amdgcn_ds_bpermute((4 * rg + i) * 4, (int)sreg[r]);
      if constexpr (FMT == kNF4)
        rowv[i] = nf4_dword_to_bf16_t16(lds0, wreg[r][i], reg2, __uint_as_float(sc));
      else
        rowv[i] = mx_dword_to_bf16(wreg[r][i], e8m0_to_f32(sc));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned r0 = rowv[0][j], r1 = rowv[1][j], r2 = rowv[2][j], r3 = rowv[3][j];
      const unsigned lo01 = __builtin_amdgcn_perm(r1, r0, 0x05040100u);   // k even: rows 0, 1
      const unsigned lo23 = __builtin_amdgcn_perm(r3, r2, 0x05040100u);
      const unsigned hi01 = __builtin_amdgcn_perm(r1, r0, 0x07060302u);   // k odd
      const unsigned hi23 = __builtin_amdgcn_perm(r3, r2, 0x07060302u);
      const int k_lo = kc * 8 + 2 * j, k_hi = k_lo + 1;
      *reinterpret_cast<uint2*>(bb + k_lo * 128 + ((rg >> 1) ^ pf_swz(k_lo & 15)) * 16 + (rg & 1) * 8) =
          make_uint2(lo01, lo23);
      *reinterpret_cast<uint2*>(bb + k_hi * 128 + ((rg >> 1) ^ pf_swz(k_hi & 15)) * 16 + (rg & 1) * 8) =
          make_uint2(hi01, hi23);
    }
  };

  auto mma = [&](auto RI, const char* stage) {
    const char* bb = bbuf_of(RI);
    u32x4_t wv[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) wv[kk] = *reinterpret_cast<const u32x4_t*>(bb + b_wave + a_off[kk]);
    u32x4_t av[2][kMT];
    auto read = [&](int buf, int kk) {
#pragma unroll
      for (int i = 0; i < kMT; ++i)
        av[buf][i] = *reinterpret_cast<const u32x4_t*>(stage + a_off[kk] + i * 4096);
    };
    read(0, 0);
    read(1, 1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kMT; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(wv[kk]), as_bf16x8(av[kk & 1][i]),
                                                          acc[i], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (kk + 2 < 4) read(kk & 1, kk + 2);
    }
  };

  auto compute = [&](auto RI, auto DF, const char* stage) {
    constexpr int r = decltype(RI)::value;
    if constexpr (decltype(DF)::value) {
      decode(std::integral_constant<int, (r + 1) % kS>{});
      __builtin_amdgcn_sched_barrier(0);
      mma(RI, stage);
    } else {
      mma(RI, stage);
      __builtin_amdgcn_sched_barrier(0);
      decode(std::integral_constant<int, (r + 1) % kS>{});
    }
    if (ring_last[r]) {
      const PfTile t = ring_t[r];
      const int rows = uniform(t.rows);
      const int c_l = t.n0 + wave * 32 + 4 * h;
      uint16_t* o = out + (int64_t)(t.row0 + l32) * p.ldo + c_l;
#pragma unroll
      for (int i = 0; i < kMT; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if (i * 32 + l32 < rows && c_l + 8 * g < p.K) {
            uint2 v;
            v.x = bf16x2_bits(acc[i][4 * g + 0], acc[i][4 * g + 1]);
            v.y = bf16x2_bits(acc[i][4 * g + 2], acc[i][4 * g + 3]);
            *reinterpret_cast<uint2*>(o + (int64_t)i * 32 * p.ldo + 8 * g) = v;
          }
        }
        acc[i] = f32x16_t{};
      }
    }
  };

  int f = 0;
  auto step = [&](auto RI, auto DF) {
    constexpr int r = decltype(RI)::value;
    constexpr int rf = (r + kS - 1) % kS;
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<(kS - 2) * kGroupLoads>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(std::integral_constant<int, rf>{}, stage_of(std::integral_constant<int, rf>{}),
          f + kS - 1 < F);
    __builtin_amdgcn_sched_barrier(0);
    compute(RI, DF, stage_of(RI));
    return ++f < F;
  };

  issue(std::integral_constant<int, 0>{}, s_a0, true);
  issue(std::integral_constant<int, 1>{}, s_a1, F > 1);
  issue(std::integral_constant<int, 2>{}, s_a2, F > 2);
  if constexpr (FMT == kNF4) __syncthreads();  // pair table complete
  decode(std::integral_constant<int, 0>{});
  if (wave < kWaves / 2) {
    auto st = [&](auto RI) { return step(RI, std::true_type{}); };
    while (StepUnroll<0, kS>::run(st)) {
    }
  } else {
    auto st = [&](auto RI) { return step(RI, std::false_type{}); };
    while (StepUnroll<0, kS>::run(st)) {
    }
  }
  // the past-the-end direct-to-LDS loads (zero-size resources) still write
  // their LDS slots: let them land before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt(0);
}

// ================================================================= dgrad ==

struct DgradArgs {
  const uint16_t* g;        // [T, ldg] bf16 (grad_out)
  int64_t ldg;
  const uint8_t* B;
  int64_t sbe, sbn;
  const void* S;
  int64_t sse, ssn;
  const int32_t* eids;
  const int32_t* t_row0;
  const int32_t* t_rows;
  const int32_t* t_group;
  int n_mtiles;
  int64_t N, K;
  uint16_t* out;            // [T, ldo] bf16
  int64_t ldo;
};

constexpr int kDgBK = 128;  // output k-tile

// Weight tile for one 64-wide n-step: 64 rows x kDgBK k. Thread t owns rows
// 4 (t / 16) .. +3 and k-elements [8 (t % 16), +8): four packed dwords, one
// scale per row. Stored k-major (transposed) so the MFMA B operand (8
// consecutive n for one k) is a single 16-byte LDS read.
template <int FMT>
struct DgRegs {
  unsigned w[4];
  float s[4];
};

template <int FMT>
__device__ __forceinline__ float dg_scale(const DgradArgs& p, int64_t e, int64_t n, int64_t k) {
  if constexpr (FMT == kNF4) {
    return static_cast<const float*>(p.S)[e * p.sse + n * p.ssn + (k >> 6)];
  } else {
    return e8m0_to_f32(static_cast<const uint8_t*>(p.S)[e * p.sse + n * p.ssn + (k >> 5)]);
  }
}

template <int FMT>
__device__ __forceinline__ void load_b_dg(DgRegs<FMT>& r, const DgradArgs& p, int64_t e,
                                          int64_t n0, int64_t k0) {
  const int rg = threadIdx.x >> 4, kc = threadIdx.x & 15;
  const int64_t k = k0 + kc * 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n = n0 + rg * 4 + i;
    if (n < p.N && k < p.K) {
      r.w[i] = *reinterpret_cast<const unsigned*>(p.B + e * p.sbe + n * p.sbn + (k >> 1));
      r.s[i] = dg_scale<FMT>(p, e, n, k);
    } else {
      r.w[i] = 0u;
      r.s[i] = 0.0f;
    }
  }
}

template <int FMT>
__device__ __forceinline__ void store_b_dg(const DgRegs<FMT>& r, const float2* tab,
                                           uint16_t* lds) {
  const int rg = threadIdx.x >> 4, kc = threadIdx.x & 15;
  const unsigned lane_off = (unsigned)(threadIdx.x & 31) * 8u;
  u32x4_t rowv[4];  // per row: 8 elements as 4 bf16 pairs
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (FMT == kNF4) rowv[i] = nf4_dword_to_bf16(tab, r.w[i], lane_off, r.s[i]);
    else rowv[i] = mx_dword_to_bf16(r.w[i], r.s[i]);
  }
  // transpose 4 rows x 8 k -> 8 k-rows of 4 consecutive n (8 bytes each)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // pair j holds k = 2j (low half) and 2j+1 (high half) of each row
    const unsigned r0 = rowv[0][j], r1 = rowv[1][j], r2 = rowv[2][j], r3 = rowv[3][j];
    const unsigned lo01 = __builtin_amdgcn_perm(r1, r0, 0x05040100u);  // k=2j: rows 0,1
    const unsigned lo23 = __builtin_amdgcn_perm(r3, r2, 0x05040100u);
    const unsigned hi01 = __builtin_amdgcn_perm(r1, r0, 0x07060302u);  // k=2j+1
    const unsigned hi23 = __builtin_amdgcn_perm(r3, r2, 0x07060302u);
    const int k_lo = kc * 8 + 2 * j;
    *reinterpret_cast<uint2*>(lds + k_lo * kLdsRow + rg * 4) = make_uint2(lo01, lo23);
    *reinterpret_cast<uint2*>(lds + (k_lo + 1) * kLdsRow + rg * 4) = make_uint2(hi01, hi23);
  }
}

template <int FMT, int BM>
__global__ void __launch_bounds__(kThreads, 1) k_gemm_dgrad(const DgradArgs p) {
  constexpr int WM = WaveGrid<BM>::WM, WN = 4 / WM;
  constexpr int MT = BM / WM / 16, NT = kDgBK / WN / 16;
  constexpr int AP = (BM * 8 + kThreads - 1) / kThreads;
  __shared__ float2 s_tab[FMT == kNF4 ? kPairEntries : 1];
  __shared__ __attribute__((aligned(16))) uint16_t s_a[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t s_b[2][kDgBK * kLdsRow];
  if constexpr (FMT == kNF4) init_pair_table(s_tab, nf4_lut_lane());

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l16 = lane & 15, q = lane >> 4;
  const int64_t k_tiles = (p.K + kDgBK - 1) / kDgBK;
  const int64_t total = (int64_t)p.n_mtiles * k_tiles;
  const int64_t nsteps = (p.N + 63) >> 6;

  for (int64_t t = blockIdx.x; t < total; t += gridDim.x) {
    const int mt = (int)(t / k_tiles);
    const int64_t k0 = (t - (int64_t)mt * k_tiles) * kDgBK;
    const int64_t row0 = p.t_row0[mt];
    const int rows = p.t_rows[mt];
    const int64_t e = p.eids[p.t_group[mt]];

    u32x4_t areg[AP];
    DgRegs<FMT> breg;
    __syncthreads();
    load_a_tile<BM>(areg, p.g, p.ldg, row0, rows, 0, p.N);
    load_b_dg<FMT>(breg, p, e, 0, k0);
    store_a_tile<BM>(areg, s_a[0]);
    store_b_dg<FMT>(breg, s_tab, s_b[0]);
    __syncthreads();

    f32x4_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int64_t ns = 0; ns < nsteps; ++ns) {
      const int cur = (int)(ns & 1);
      const bool more = ns + 1 < nsteps;
      if (more) {
        load_a_tile<BM>(areg, p.g, p.ldg, row0, rows, (ns + 1) * 64, p.N);
        load_b_dg<FMT>(breg, p, e, (ns + 1) * 64, k0);
      }
      const uint16_t* la = s_a[cur];
      const uint16_t* lb = s_b[cur];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u32x4_t bop[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j)
          bop[j] = *reinterpret_cast<const u32x4_t*>(
              lb + ((wn * NT + j) * 16 + l16) * kLdsRow + kk * 32 + q * 8);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const u32x4_t aop = *reinterpret_cast<const u32x4_t*>(
              la + ((wm * MT + i) * 16 + l16) * kLdsRow + kk * 32 + q * 8);
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[i][j] = mfma(aop, bop[j], acc[i][j]);
        }
      }
      if (more) {
        store_a_tile<BM>(areg, s_a[cur ^ 1]);
        store_b_dg<FMT>(breg, s_tab, s_b[cur ^ 1]);
      }
      __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int64_t k = k0 + (wn * NT + j) * 16 + l16;
        if (k >= p.K) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = (wm * MT + i) * 16 + 4 * q + r;
          if (m < rows) p.out[(row0 + m) * p.ldo + k] = f32_to_bf16_bits(acc[i][j][r]);
        }
      }
    }
  }
}

// ================================================================== host ==

struct DevInfo {
  int cus = 0;
};

DevInfo g_dev[64];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (g_dev[dev].cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    g_dev[dev].cus = cus;
  }
  return g_dev[dev].cus;
}

int64_t clamp_grid(int64_t work, int64_t cap) { return work < cap ? (work > 0 ? work : 1) : cap; }

// Launch one decode-kernel instance with `lds` bytes of dynamic LDS.
template <int FMT, int CPW, int T, int W, int PA, int S>
int launch_decode_inst(const FwdArgs& p, dim3 grid, int lds, hipStream_t stream) {
  static int configured_dev = -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -2;
  if (configured_dev != dev) {   // allow more than the default 64 KiB of dynamic LDS
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_decode_fwd<FMT, CPW, T, W, PA, S>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
      return -2;
    configured_dev = dev;
  }
  hipLaunchKernelGGL((k_decode_fwd<FMT, CPW, T, W, PA, S>), grid, dim3(64 * W), lds, stream, p);
  return 0;
}

// The kernel-argument ids of a launch (empty: the kernels read the tables).
const GemvIds& gemv_ids_of(const FwdArgs& p) {
  static const GemvIds empty{};
  return p.ids_inline ? *p.ids_inline : empty;
}

// One-row decode launch (k_gemv_nf4, k_gemv_mx): every group exactly one
// row and at most four pieces per lane (NF4 K <= 8192). Row steps per wave:
// enough for about one workgroup per CU over the launch's rows, at most six
// (measured on MI355X at batch 1: Qwen3-30B-A3B gate_up 6 and down 4,
// GPT-OSS-20B gate_up 6 and down 3 per wave were the fastest of 1..12;
// more, smaller workgroups and 1024-thread workgroups were slower). Returns
// 1 when the launch is not for it.

template <int FMT, int LR, int PPL, int RPW, bool ROWS>
int launch_gemv_inst(const FwdArgs& p, hipStream_t stream) {
  const int64_t rows_wg = 8 * RPW * (64 / LR);
  const int64_t gx = (p.N + rows_wg - 1) / rows_wg;
  if (gx > 0x7FFFFFFF) return -1;
  const dim3 grid((unsigned)gx, (unsigned)p.G, 1);
  if constexpr (FMT == kNF4)
    hipLaunchKernelGGL((k_gemv_nf4<LR, PPL, RPW, false, ROWS>), grid, dim3(512),
                       8 * kPairEntries, stream, p, 0, gemv_ids_of(p));
  else
    hipLaunchKernelGGL((k_gemv_mx<LR, PPL, RPW>), grid, dim3(512), 0, stream, p, gemv_ids_of(p));
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

template <int FMT, int LR, int PPL, bool ROWS = false>
int launch_gemv_rpw(const FwdArgs& p, int rpw, hipStream_t stream) {
  switch (rpw) {
    case 2: return launch_gemv_inst<FMT, LR, PPL, 2, ROWS>(p, stream);
    case 3: return launch_gemv_inst<FMT, LR, PPL, 3, ROWS>(p, stream);
    case 4: return launch_gemv_inst<FMT, LR, PPL, 4, ROWS>(p, stream);
    default: return launch_gemv_inst<FMT, LR, PPL, 6, ROWS>(p, stream);
  }
}

// Slots per row of the one-row order: NF4 follows onerow_slots (the fused
// FFN's decode units share it); MXFP4 takes whichever of 32 and 64 leaves
// fewer idle lanes (GPT-OSS-20B K = 2880: 90 pieces, 3 x 32 lanes).
template <int FMT>
int gemv_slots(int64_t pr) {
  if (FMT == kNF4) return pr <= 32 ? 32 : 64;
  return 32 * ((pr + 31) / 32) < 64 * ((pr + 63) / 64) ? 32 : 64;
}

// The multi-row NF4 GEMV (k_gemv_nf4 with ROWS) takes decode launches whose
// groups have at most four rows at 1024 < K <= 2048 (one 16-byte piece per
// lane and row, 64 lanes a row), at most two rows at K <= 1024 (32 lanes a
// row); larger groups, and larger K, keep the split-table kernels. The class
// follows the largest group and K only, so a group's bits never depend on
// the other groups of the launch. Measured on MI355X at Qwen3-30B-A3B shapes
// (per launch, uniform top-8 of 128 experts): batch 2 gate_up 10.1 -> 8.9 us,
// down (K = 768) 8.7 -> 7.2 us; batch 4 (largest group 3) gate_up 20.2 ->
// 15.4 us. Where they lose: K = 768 at groups of 3..4 rows over many groups
// (batch 16 layers whose largest group is 4: down 26.5 against 30.9 us), and
// groups of 5..8 rows at K = 2048 (16 experts, 8 tokens: 14.3 against
// 24.1 us).
constexpr int kGemvMaxRows = 4;       // 1024 < K <= 2048
constexpr int kGemvMaxRowsNarrow = 2; // K <= 1024

// Whether an NF4 decode launch of groups of more than one row takes the GEMV.
bool gemv_nf4_takes_rows(int max_m, int64_t K) {
  if (max_m <= 1 || K % 64 != 0 || K > 2048) return false;
  return max_m <= (K > 1024 ? kGemvMaxRows : kGemvMaxRowsNarrow);
}
bool gemv_nf4_takes(const FwdArgs& p) {
  const bool has_ro = p.ids_inline ? p.ids_inline->has_ro != 0 : p.row_off != nullptr;
  return has_ro && gemv_nf4_takes_rows(p.max_m, p.K);
}

// Whether launch_gemv<FMT> leaves p to another kernel class (returns 1
// without launching anything).
template <int FMT>
bool gemv_refuses(const FwdArgs& p) {
  if (p.K <= 0 || p.K % (FMT == kNF4 ? 64 : 32) != 0 || p.N <= 0 || p.G <= 0) return true;
  const int64_t pr = p.K / 32;
  const int lr = gemv_slots<FMT>(pr);
  const int64_t ppl = (pr + lr - 1) / lr;
  if (ppl > 4) return true;
  // 32-bit row offsets inside the expert's resources
  const int64_t sbytes = FMT == kNF4 ? 4 : 1;
  if (p.N * p.sbn > 0x7FFFFFFF || p.N * p.ssn * sbytes > 0x7FFFFFFF) return true;
  if (p.max_m > 1 && (FMT != kNF4 || !gemv_nf4_takes(p) || ppl != 1)) return true;
  return false;
}

template <int FMT>
int launch_gemv(const FwdArgs& p, hipStream_t stream) {
  if (gemv_refuses<FMT>(p)) return 1;
  const int64_t pr = p.K / 32;
  const int lr = gemv_slots<FMT>(pr);
  const int64_t ppl = (pr + lr - 1) / lr;
  const int cus = device_cus();
  if (cus <= 0) return -2;
  // row steps per wave: about one workgroup per CU over the launch's rows
  const int64_t per_step = (int64_t)cus * 8 * (64 / lr);
  const int64_t want = ((int64_t)p.G * p.N + per_step - 1) / per_step;
  const int rpw = want <= 2 ? 2 : want <= 3 ? 3 : want <= 4 ? 4 : 6;
  if constexpr (FMT == kNF4) {
    if (p.max_m > 1) {   // ppl == 1 here
      if (lr == 32) return launch_gemv_rpw<FMT, 32, 1, true>(p, rpw, stream);
      return launch_gemv_rpw<FMT, 64, 1, true>(p, rpw, stream);
    }
  }
  if (lr == 32) {
    if constexpr (FMT == kNF4) return launch_gemv_rpw<FMT, 32, 1>(p, rpw, stream);   // pr <= 32
    switch (ppl) {
      case 1: return launch_gemv_rpw<FMT, 32, 1>(p, rpw, stream);
      case 2: return launch_gemv_rpw<FMT, 32, 2>(p, rpw, stream);
      case 3: return launch_gemv_rpw<FMT, 32, 3>(p, rpw, stream);
      default: return launch_gemv_rpw<FMT, 32, 4>(p, rpw, stream);
    }
  }
  switch (ppl) {
    case 1: return launch_gemv_rpw<FMT, 64, 1>(p, rpw, stream);
    case 2: return launch_gemv_rpw<FMT, 64, 2>(p, rpw, stream);
    case 3: return launch_gemv_rpw<FMT, 64, 3>(p, rpw, stream);
    default: return launch_gemv_rpw<FMT, 64, 4>(p, rpw, stream);
  }
}

// pa: LDS-staged activation pieces per thread (0: register operands);
// sets: NF4 row sets (0: one-row groups on the fp32 FMA path, 2 when a group
// has more than 8 rows)
template <int FMT, int CPW, int T>
int launch_decode_pa(const FwdArgs& p, dim3 grid, int pa, int sets, int lds, hipStream_t stream) {
  constexpr int W = 8;
  if constexpr (FMT == kNF4) {
    if (sets == 0) {
      switch (pa) {
        case 1: return launch_decode_inst<FMT, CPW, T, W, 1, 0>(p, grid, lds, stream);
        case 2: return launch_decode_inst<FMT, CPW, T, W, 2, 0>(p, grid, lds, stream);
        case 4: return launch_decode_inst<FMT, CPW, T, W, 4, 0>(p, grid, lds, stream);
        default: return -1;
      }
    }
  }
  switch (pa) {
    case 1: return launch_decode_inst<FMT, CPW, T, W, 1, 1>(p, grid, lds, stream);
    case 2: return launch_decode_inst<FMT, CPW, T, W, 2, 1>(p, grid, lds, stream);
    case 4: return launch_decode_inst<FMT, CPW, T, W, 4, 1>(p, grid, lds, stream);
    case 8:
      if constexpr (FMT != kNF4) return launch_decode_inst<FMT, CPW, T, W, 8, 1>(p, grid, lds, stream);
      return -1;
    default:
      if constexpr (FMT == kNF4)
        if (sets == 2) return launch_decode_inst<FMT, CPW, T, W, 0, 2>(p, grid, lds, stream);
      return launch_decode_inst<FMT, CPW, T, W, 0, 1>(p, grid, lds, stream);
  }
}

// LDS staging of a decode launch's activations (eight waves per workgroup):
// NF4 groups of at most two rows (beside the 64 KiB split table), at most 4
// pieces of 16 bytes per thread; MXFP4 groups whose padded rows fit two
// workgroups per CU, at most 8 pieces per thread. Returns the pieces per
// thread (0: operands load into registers) and the staged bytes.
template <int FMT>
int decode_stage(int64_t K, int64_t max_m, int64_t* a_bytes) {
  constexpr int64_t kThreadsD = 64 * 8;
  const int64_t pieces = max_m * (K / 8);
  // layout of decode_unit (one NF4 row: widened to fp32, 32 bytes a piece)
  const int64_t bytes = ((FMT == kNF4 && max_m == 1 ? 2 : 1) * pieces + K / 32 + 1) * 16;
  const bool stage = FMT == kNF4 ? max_m <= 2 && pieces <= 4 * kThreadsD
                                 : bytes + 64 <= 80 * 1024 && pieces <= 8 * kThreadsD;
  *a_bytes = stage ? bytes : 0;
  if (!stage) return 0;
  return pieces <= kThreadsD ? 1 : pieces <= 2 * kThreadsD ? 2 : pieces <= 4 * kThreadsD ? 4 : 8;
}

// Decode launch: one workgroup of eight waves per unit (group, 16 kT rows).
// Groups of at most two rows stage their activations in LDS; larger ones load
// them into registers. NF4 runs at most two chunks per wave per round (its
// absmax run load covers two), MXFP4 up to four.
template <int FMT, int kT>
int launch_decode_t(const FwdArgs& p, hipStream_t stream) {
  constexpr int kW = 8;
  const int64_t per_wave = ((p.K + 127) / 128 + kW - 1) / kW;
  const int64_t n_units = (p.N + 16 * kT - 1) / (16 * kT);
  if (p.G <= 0 || n_units == 0) return 0;
  if ((int64_t)p.G * n_units > 0x7FFFFFFF || n_units > 0x7FFFFFFF) return -1;
  if (p.G > 65535) return -1;   // grid rows (launch_decode splits larger calls)
  const dim3 grid((unsigned)n_units, (unsigned)p.G, 1);
  int64_t a_bytes = 0;
  const int pa = decode_stage<FMT>(p.K, p.max_m, &a_bytes);
  const bool stage = pa > 0;
  const int sets = FMT != kNF4 ? 1 : p.max_m > 8 ? 2 : (p.max_m == 1 && pa > 0) ? 0 : 1;
  if ((FMT == kNF4 && (sets == 0 || gemv_nf4_takes(p))) || (FMT == kMX && p.max_m == 1)) {
    // one-row groups: the row-major GEMV (NF4: same bits as decode_unit's
    // one-row form)
    const int rc = launch_gemv<FMT>(p, stream);
    if (rc <= 0) return rc;
  }
  const int64_t red = (int64_t)kW * kT * (sets > 0 ? sets : 1) * 64 * 16;
  const int64_t table = FMT == kNF4 ? kSplitTabBytes : 0;
  int64_t lds = table + kDecodeFlagBytes + (stage ? a_bytes : 0) + 64;
  if (lds < red) lds = red;
  if (lds > 160 * 1024) return -1;
  if (per_wave <= 1) return launch_decode_pa<FMT, 1, kT>(p, grid, pa, sets, (int)lds, stream);
  if constexpr (FMT == kNF4) {
    // two row sets: one chunk per wave and round (two spill 128 VGPRs)
    if (sets == 2) return launch_decode_pa<FMT, 1, kT>(p, grid, pa, sets, (int)lds, stream);
    return launch_decode_pa<FMT, 2, kT>(p, grid, pa, sets, (int)lds, stream);
  } else {
    if (per_wave <= 2) return launch_decode_pa<FMT, 2, kT>(p, grid, pa, 1, (int)lds, stream);
    if (per_wave <= 3 || !stage)   // register operands: 3 chunks per round fit 128 VGPRs
      return launch_decode_pa<FMT, 3, kT>(p, grid, pa, 1, (int)lds, stream);
    return launch_decode_pa<FMT, 4, kT>(p, grid, pa, 1, (int)lds, stream);
  }
}

// Chunks per wave of a k_decode_fwd launch (its rounds' length).
template <int FMT>
int decode_cpw(int64_t K, int64_t max_m) {
  constexpr int kW = 8;
  const int64_t per_wave = ((K + 127) / 128 + kW - 1) / kW;
  int64_t a_bytes = 0;
  const bool stage = decode_stage<FMT>(K, max_m, &a_bytes) > 0;
  if (per_wave <= 1) return 1;
  if (FMT == kNF4) return max_m > 8 ? 1 : 2;   // as launch_decode_t
  if (per_wave <= 2) return 2;
  if (per_wave <= 3 || !stage) return 3;
  return 4;
}

// Row-streaming decode (k_decode_rows) for a launch whose k_decode_fwd
// form needs one round per wave (so the two kernels' bits agree); returns 1
// when this launch is not for it.
template <int FMT, int W, int T, int S, int CPW, int R, int P, bool AB>
int launch_rows_inst(const FwdArgs& p, int lds, hipStream_t stream) {
  static int configured_dev = -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -2;
  if (configured_dev != dev) {
    if (hipFuncSetAttribute(
            reinterpret_cast<const void*>(&k_decode_rows<FMT, W, T, S, CPW, R, P, AB>),
            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
      return -2;
    configured_dev = dev;
  }
  const dim3 grid((unsigned)((p.N + 16 * W * T - 1) / (16 * W * T)), (unsigned)p.G, 1);
  hipLaunchKernelGGL((k_decode_rows<FMT, W, T, S, CPW, R, P, AB>), grid, dim3(64 * W), lds, stream,
                     p);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// ring: kCpw x kR chunks per wave
template <int FMT, int W, int S, int P>
int launch_rows_cpw(const FwdArgs& p, int cpw, int lds, hipStream_t stream) {
  // (fewer than 8 chunks: k_decode_fwd runs one chunk per wave)
  if (cpw != 1) return 1;
  // absmax as whole 16-row blocks where a block fits one 1 KiB load, its
  // rows are a multiple of 4 floats and the loads are aligned
  const bool ab = p.ssn % 4 == 0 && p.ssn <= 16 && p.sse % 4 == 0 &&
                  reinterpret_cast<uintptr_t>(p.S) % 16 == 0;
  if (ab) return launch_rows_inst<FMT, W, 2, S, 1, 2, P, true>(p, lds, stream);
  return launch_rows_inst<FMT, W, 2, S, 1, 2, P, false>(p, lds, stream);
}

// Taken for NF4 launches of groups of 2..8 rows whose K gives k_decode_fwd's
// eight waves fewer than eight chunks (K <= 768: idle waves there). Measured
// on MI355X, Qwen3-30B-A3B down projection (K = 768): batch 4 1241 -> 1721
// GB/s, batch 16 1405 -> 2267 GB/s; at K = 2048 and for MXFP4 (K = 2880)
// the split-K kernel stays faster, and two row sets spill here.
template <int FMT>
int launch_rows(const FwdArgs& p, hipStream_t stream) {
  if constexpr (FMT != kNF4) {
    return 1;
  } else {
  if (p.max_m < 2 || p.max_m > 8 || p.G <= 0 || p.G > 65535) return 1;
  const int64_t nchunks = (p.K + 127) / 128;
  if (nchunks >= 8) return 1;
  const int cpw = decode_cpw<FMT>(p.K, p.max_m);
  if (nchunks > 8 * cpw) return 1;                     // k_decode_fwd takes rounds
  const int64_t kslices = p.K / 8;
  const int64_t pieces = (int64_t)p.max_m * kslices;
  const int64_t lds = (FMT == kNF4 ? kSplitTabBytes : 0) + (pieces + kslices / 4 + 1) * 16 + 64;
  if (lds > 160 * 1024) return 1;
  const int sets = FMT == kNF4 && p.max_m > 8 ? 2 : 1;
  const bool two = lds <= 80 * 1024;                  // two workgroups of 8 waves per CU
  const int64_t threads = two ? 512 : 1024;
  const int pp = (int)((pieces + threads - 1) / threads);
  if (pp > 8) return 1;
  const int P = pp <= 2 ? 2 : pp <= 4 ? 4 : 8;
  (void)sets;
  const FwdArgs& q = p;
  if (two) return P == 2 ? launch_rows_cpw<FMT, 8, 1, 2>(q, cpw, (int)lds, stream)
                 : P == 4 ? launch_rows_cpw<FMT, 8, 1, 4>(q, cpw, (int)lds, stream)
                          : launch_rows_cpw<FMT, 8, 1, 8>(q, cpw, (int)lds, stream);
  return P == 2 ? launch_rows_cpw<FMT, 16, 1, 2>(q, cpw, (int)lds, stream)
         : P == 4 ? launch_rows_cpw<FMT, 16, 1, 4>(q, cpw, (int)lds, stream)
                  : launch_rows_cpw<FMT, 16, 1, 8>(q, cpw, (int)lds, stream);
  }
}

template <int CPW, int R, bool LS>
int launch_stream_inst(const FwdArgs& p, dim3 grid, int upg, int per_wg, int lds,
                       hipStream_t stream) {
  static int configured_dev = -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -2;
  if (configured_dev != dev) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_decode_stream<CPW, R, LS>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
      return -2;
    configured_dev = dev;
  }
  hipLaunchKernelGGL((k_decode_stream<CPW, R, LS>), grid, dim3(512), lds, stream, p, upg, per_wg);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Unit walks for batched decode: k_decode_stream_nf4 for NF4 groups of 2..8
// rows at 1024 < K <= 2048 (each workgroup walking at least 4 units), and
// k_decode_stream for batched MXFP4 launches whose
// k_decode_fwd form runs three chunks per wave in one round (so the bits
// agree; GPT-OSS: K = 2880). Each group gets about 256 / G workgroups (one
// per CU), each a contiguous range of units. MXFP4 takes it when every
// workgroup walks at least 4 units: measured on MI355X at GPT-OSS-20B
// shapes against the per-unit kernel, batch 3 / 4 gate_up 24.6 / 30.5 ->
// 22.9 / 27.5 us, batch 6 / 8 down 22.5 / 25.1 -> 20.7 / 22.8 us, batch 64
// gate_up 88.2 -> 61.9 us; walks of 2..3 units (batch 2 down) run 2 %
// slower.
// Returns 1 when the launch is not for it.
template <int FMT>
int launch_stream(const FwdArgs& p, hipStream_t stream) {
  if constexpr (FMT != kMX) {
    // NF4: k_decode_stream_nf4, 16-row units, one unit in flight per team.
    // Its workgroups are dealt to the groups in equal shares, so where groups
    // may be empty (device routing: the launch covers a bound of the active
    // groups) their shares would idle: the per-unit kernel spreads the units
    // instead (Qwen3 batch 16 routed FFN: 81.3 -> 74.8 us)
    if (p.sparse_groups) return 1;
    if (p.max_m < 2 || p.max_m > 8 || p.row_off == nullptr || p.G <= 0 || p.G > 65535) return 1;
    const int64_t nchunks = (p.K + 127) / 128;
    if (decode_cpw<FMT>(p.K, p.max_m) != 2 || nchunks > 16) return 1;   // 1024 < K <= 2048
    const int64_t kslices = p.K / 8;
    const int64_t lds = kSplitTabBytes + ((int64_t)p.max_m * kslices + kslices / 4 + 1) * 16 +
                        64 + 2 * 8 * 64 * 16;
    if (lds > 160 * 1024) return 1;
    const int64_t upg = (p.N + 15) / 16;
    int64_t wpg = 256 / p.G;
    if (wpg < 1) wpg = 1;
    const int64_t per_wg = (upg + wpg - 1) / wpg;
    if (per_wg < 4) return 1;
    wpg = (upg + per_wg - 1) / per_wg;
    // Whole workgroups per group leave CUs idle for some group counts
    // (G = 86 on 256 CUs: 2 per group, 172 busy). The walk's time follows
    // its longest range (per_wg units), the per-unit kernel's the total
    // (it spreads every unit over every CU); measured at Qwen3 gate_up
    // shapes (G = 60..120, 1..4 rows): walk ~ 0.96 us x per_wg + 10.7 us,
    // per-unit ~ 5.4 ns x units + 7.9 us, so the walk runs where
    // units >= CUs x (0.7 per_wg + 2).
    const int cus = device_cus();
    if (cus <= 0) return -2;
    if (upg * p.G * 10 < (int64_t)cus * (7 * per_wg + 20)) return 1;
    const dim3 grid((unsigned)wpg, (unsigned)p.G, 1);
    static int configured_dev = -1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -2;
    if (configured_dev != dev) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_decode_stream_nf4<1, 1>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
        return -2;
      configured_dev = dev;
    }
    hipLaunchKernelGGL((k_decode_stream_nf4<1, 1>), grid, dim3(1024), (int)lds, stream, p,
                       (int)upg, (int)per_wg);
    return hipGetLastError() == hipSuccess ? 0 : -2;
  } else {
    if (p.sparse_groups) return 1;
    if (p.max_m < 2 || p.max_m > 16 || p.row_off == nullptr || p.G <= 0 || p.G > 65535) return 1;
    const int64_t nchunks = (p.K + 127) / 128;
    if (decode_cpw<FMT>(p.K, p.max_m) != 3 || nchunks > 8 * 3) return 1;
    const int64_t kslices = p.K / 8;
    const int64_t lds = ((int64_t)p.max_m * kslices + kslices / 4 + 1) * 16 + 64 + 8 * 2 * 64 * 16;
    if (lds > 160 * 1024) return 1;
    const int64_t upg = (p.N + 31) / 32;
    int64_t wpg = 256 / p.G;
    if (wpg < 1) wpg = 1;
    const int64_t per_wg = (upg + wpg - 1) / wpg;
    if (per_wg < 4) return 1;
    wpg = (upg + per_wg - 1) / per_wg;
    const dim3 grid((unsigned)wpg, (unsigned)p.G, 1);
    // a ring of two units per wave: measured against three, four and five
    // (deeper rings run 1-5 % slower), and against two workgroups per CU
    // where the staged rows allow it (no faster)
    // Scale blocks through LDS where a unit's block fits 3 KiB and the
    // 16-byte loads of it are aligned (every contiguous [E, N, K / 32] stack
    // of K <= 3072 in a 16-byte aligned buffer).
    const bool lds_scales = p.ssn <= 96 && p.sse % 16 == 0 &&
                            reinterpret_cast<uintptr_t>(p.S) % 16 == 0 &&
                            lds + 2 * 3072 <= 160 * 1024;
    if (lds_scales)
      return launch_stream_inst<3, 2, true>(p, grid, (int)upg, (int)per_wg, (int)(lds + 2 * 3072),
                                            stream);
    return launch_stream_inst<3, 2, false>(p, grid, (int)upg, (int)per_wg, (int)lds, stream);
  }
}

// Unit height: 32 rows, or 16 for single-row MXFP4 groups (more workgroups
// for a stream that needs little decode work per byte).
// Groups go to the grid's rows, at most 65535 per launch: larger calls run as
// several launches over consecutive group ranges.
template <int FMT>
int launch_decode(const FwdArgs& p, hipStream_t stream) {
  if (FMT == kNF4 && gemv_nf4_takes(p) && p.G <= 65535) {
    const int rc = launch_gemv<FMT>(p, stream);
    if (rc <= 0) return rc;
  }
  {
    const int rc = launch_rows<FMT>(p, stream);
    if (rc <= 0) return rc;
  }
  {
    const int rc = launch_stream<FMT>(p, stream);
    if (rc <= 0) return rc;
  }
  for (int g0 = 0; g0 < p.G; g0 += 65535) {
    FwdArgs q = p;
    q.G = p.G - g0 < 65535 ? p.G - g0 : 65535;
    q.eids = p.eids + g0;
    if (p.row_off) {
      q.row_off = p.row_off + ((int64_t)g0 << p.ro_shift);   // absolute row offsets
    } else {                        // group g is row g
      q.a = p.a + (int64_t)g0 * p.lda;
      q.out = p.out + (int64_t)g0 * p.ldo;
    }
    const int rc = FMT == kMX && p.max_m == 1 ? launch_decode_t<FMT, 1>(q, stream)
                                              : launch_decode_t<FMT, 2>(q, stream);
    if (rc) return rc;
  }
  return 0;
}

// Fused FFN decode launch (every group at most 16 rows). Phase shapes:
// gate/up over K, down over H; the chunk split per wave follows each K.
// Sync words and per-call values of a fused FFN launch.
struct FfnSync {
  uint32_t* words;
  uint32_t epoch;      // nonzero; differs between consecutive launches
  int spin_limit;
};

// Per-process launch counter for the flag epochs, and the spin limit of
// later launches (gnf4_hip_ffn_set_spin_limit).
std::atomic<uint32_t> g_ffn_epoch{0};
std::atomic<int> g_ffn_spin_limit{kFfnSpinLimit};

uint32_t next_ffn_epoch() {
  uint32_t e = g_ffn_epoch.fetch_add(1, std::memory_order_relaxed) + 1;
  if (e == 0) e = g_ffn_epoch.fetch_add(1, std::memory_order_relaxed) + 1;   // 0 means clear
  return e;
}

template <int CPW1, int CPW2, int PA, int S>
int launch_ffn_inst(const FwdArgs& gu, const FwdArgs& dn, int64_t H, const FfnSync& fs,
                    uint32_t n_units, int lds, hipStream_t stream) {
  static int configured_dev = -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -2;
  if (configured_dev != dev) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_ffn_decode<CPW1, CPW2, PA, S>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kFfnMaxDynLds) !=
        hipSuccess)
      return -2;
    configured_dev = dev;
  }
  hipLaunchKernelGGL((k_ffn_decode<CPW1, CPW2, PA, S>), dim3(n_units), dim3(512), lds, stream,
                     gu, dn, H, fs.words, fs.epoch, fs.spin_limit);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

template <int CPW1, int CPW2>
int launch_ffn_pa(const FwdArgs& gu, const FwdArgs& dn, int64_t H, const FfnSync& fs,
                  uint32_t n_units, int pa, int sets, int lds, hipStream_t stream) {
  if (sets == 0) {
    switch (pa) {
      case 1: return launch_ffn_inst<CPW1, CPW2, 1, 0>(gu, dn, H, fs, n_units, lds, stream);
      case 2: return launch_ffn_inst<CPW1, CPW2, 2, 0>(gu, dn, H, fs, n_units, lds, stream);
      case 4: return launch_ffn_inst<CPW1, CPW2, 4, 0>(gu, dn, H, fs, n_units, lds, stream);
      default: return -1;
    }
  }
  switch (pa) {
    case 1: return launch_ffn_inst<CPW1, CPW2, 1, 1>(gu, dn, H, fs, n_units, lds, stream);
    case 2: return launch_ffn_inst<CPW1, CPW2, 2, 1>(gu, dn, H, fs, n_units, lds, stream);
    case 4: return launch_ffn_inst<CPW1, CPW2, 4, 1>(gu, dn, H, fs, n_units, lds, stream);
    default:
      if (sets == 2) return launch_ffn_inst<CPW1, CPW2, 0, 2>(gu, dn, H, fs, n_units, lds, stream);
      return launch_ffn_inst<CPW1, CPW2, 0, 1>(gu, dn, H, fs, n_units, lds, stream);
  }
}

// First stage of the one-row expert FFN (k_gemv_nf4 with the silu
// epilogue): gu.out is h. Returns 1 when the shape is not for it.
template <int LR, int PPL, int RPW, bool ROWS>
int launch_gemv_gu_inst(const FwdArgs& p, int64_t H, hipStream_t stream) {
  const int64_t cols_wg = 8 * (RPW / 2) * (64 / LR);
  const int64_t gx = (H + cols_wg - 1) / cols_wg;
  if (gx > 0x7FFFFFFF) return -1;
  hipLaunchKernelGGL((k_gemv_nf4<LR, PPL, RPW, true, ROWS>), dim3((unsigned)gx, (unsigned)p.G, 1),
                     dim3(512), 8 * kPairEntries, stream, p, (int)H, gemv_ids_of(p));
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

template <int LR, int PPL, bool ROWS = false>
int launch_gemv_gu_rpw(const FwdArgs& p, int64_t H, int rpw, hipStream_t stream) {
  switch (rpw) {
    case 2: return launch_gemv_gu_inst<LR, PPL, 2, ROWS>(p, H, stream);
    case 4: return launch_gemv_gu_inst<LR, PPL, 4, ROWS>(p, H, stream);
    default: return launch_gemv_gu_inst<LR, PPL, 6, ROWS>(p, H, stream);
  }
}

// gate_up stage of the expert FFN in the GEMV class: one-row groups, or
// groups the multi-row GEMV takes (gemv_nf4_takes). Returns 1 when the
// launch is not for it.
bool gemv_gu_refuses(const FwdArgs& p, int64_t H) {
  const int64_t pr = p.K / 32;
  const int lr = pr <= 32 ? 32 : 64;
  const int64_t ppl = (pr + lr - 1) / lr;
  if (p.K <= 0 || p.K % 64 || ppl > 4 || p.G <= 0 || p.G > 65535) return true;
  if (p.N * p.sbn > 0x7FFFFFFF || p.N * p.ssn * 4 > 0x7FFFFFFF || H > 0x7FFFFFFF) return true;
  return p.max_m > 1 && (!gemv_nf4_takes(p) || ppl != 1);
}

int launch_gemv_gu(const FwdArgs& p, int64_t H, hipStream_t stream) {
  if (gemv_gu_refuses(p, H)) return 1;
  const int64_t pr = p.K / 32;
  const int lr = pr <= 32 ? 32 : 64;
  const int64_t ppl = (pr + lr - 1) / lr;
  const bool multi = p.max_m > 1;
  const int cus = device_cus();
  if (cus <= 0) return -2;
  const int64_t per_step = (int64_t)cus * 8 * (64 / lr);
  const int64_t want = ((int64_t)p.G * p.N + per_step - 1) / per_step;
  const int rpw = want <= 2 ? 2 : want <= 4 ? 4 : 6;
  if (multi) {   // ppl == 1 here
    if (lr == 32) return launch_gemv_gu_rpw<32, 1, true>(p, H, rpw, stream);
    return launch_gemv_gu_rpw<64, 1, true>(p, H, rpw, stream);
  }
  if (lr == 32) return launch_gemv_gu_rpw<32, 1>(p, H, rpw, stream);
  switch (ppl) {
    case 1: return launch_gemv_gu_rpw<64, 1>(p, H, rpw, stream);
    case 2: return launch_gemv_gu_rpw<64, 2>(p, H, rpw, stream);
    case 3: return launch_gemv_gu_rpw<64, 3>(p, H, rpw, stream);
    default: return launch_gemv_gu_rpw<64, 4>(p, H, rpw, stream);
  }
}

// Fused expert FFN. One-row groups (the GEMV class) take two launches, the
// gate_up GEMV with the silu epilogue writing h and the down GEMV: no
// cross-workgroup hand-off, and faster than the single launch below (Qwen3
// batch 1, per layer: 9.8 against 13.4 us; gate_up -> silu -> down as
// three launches 12.6 us). The same bits either way.
int launch_ffn(const FwdArgs& gu, const FwdArgs& dn, int64_t H, const FfnSync& fs,
               hipStream_t stream) {
  if (gu.max_m == 1 && gu.G <= 65535) {
    FwdArgs d1 = dn;
    d1.max_m = 1;
    const int r1 = launch_gemv_gu(gu, H, stream);
    if (r1 < 0) return r1;
    if (r1 == 0) {
      const int r2 = launch_gemv<kNF4>(d1, stream);
      if (r2 <= 0) return r2;
      // the down GEMV refused a shape its first stage took: finish with the
      // one-row decode kernel, same bits
      return launch_decode<kNF4>(d1, stream);
    }
  }
  bool gu_only = false;
  if (gu.max_m > 1) {
    // multi-row groups: the plain forward of each stage takes the GEMV class
    // or the split-table kernels by its own K; the fused forms follow it
    const bool g1 = gemv_nf4_takes(gu), g2 = gemv_nf4_takes(dn);
    if (g1) {
      const int r1 = launch_gemv_gu(gu, H, stream);
      if (r1 <= 0) return r1 < 0 ? r1 : launch_decode<kNF4>(dn, stream);
      return -1;
    }
    // the down stage alone takes the GEMV class: the single launch below
    // runs its gate/up units only (h; with no down units they set no
    // flags), and the down GEMV follows
    if (g2) gu_only = true;
  }
  constexpr int kW = 8;
  const int64_t units =
      (int64_t)gu.G * (H / 16) + (gu_only ? 0 : (int64_t)gu.G * ((dn.N + 31) / 32));
  if (units <= 0) return 0;
  if (units > 0x7FFFFFFF) return -1;
  const int64_t kmax = gu.K > dn.K ? gu.K : dn.K;
  int64_t a_bytes = 0;
  const int pa = decode_stage<kNF4>(kmax, gu.max_m, &a_bytes);
  const int sets = gu.max_m > 8 ? 2 : (gu.max_m == 1 && pa > 0) ? 0 : 1;
  int64_t lds = kSplitTabBytes + kDecodeFlagBytes + a_bytes + 64;
  const int64_t red = (int64_t)kW * 2 * (sets > 0 ? sets : 1) * 64 * 16;
  if (lds < red) lds = red;
  if (lds > kFfnMaxDynLds) return -1;
  // chunks per wave as the plain decode launches take them (same bits)
  const bool two1 = sets != 2 && ((gu.K + 127) / 128 + kW - 1) / kW > 1;
  const bool two2 = sets != 2 && ((dn.K + 127) / 128 + kW - 1) / kW > 1;
  const uint32_t n = (uint32_t)units;
  FwdArgs d = dn;
  if (gu_only) d.N = 0;   // no down units: the gate/up units' flag rows are empty
  const int rc = two1 && two2 ? launch_ffn_pa<2, 2>(gu, d, H, fs, n, pa, sets, (int)lds, stream)
                 : two1       ? launch_ffn_pa<2, 1>(gu, d, H, fs, n, pa, sets, (int)lds, stream)
                 : two2       ? launch_ffn_pa<1, 2>(gu, d, H, fs, n, pa, sets, (int)lds, stream)
                              : launch_ffn_pa<1, 1>(gu, d, H, fs, n, pa, sets, (int)lds, stream);
  if (rc || !gu_only) return rc;
  return launch_decode<kNF4>(dn, stream);
}

// An empty kernel-argument tile table: the kernel reads the device tables.
const PwTiles& no_tiles() {
  static const PwTiles empty{};
  return empty;
}

// Workgroups per XCD range of the persistent k_prefill_w grid: one per CU
// (each walks several tiles; the pair table is built once per workgroup), or
// fewer when the XCD's range has fewer tiles.
int64_t prefill_w_per_xcd(int64_t tiles, int cus) {
  const int64_t per_x = (tiles + 7) / 8;
  const int64_t cap = cus >= 8 ? cus / 8 : 1;
  return per_x > cap ? cap : per_x;
}

template <int FMT>
int launch_fwd(const FwdArgs& p, int block_m, hipStream_t stream, const PwTiles* tt = nullptr) {
  const int cus = device_cus();
  if (cus <= 0) return -2;
  if (p.n_mtiles == 0) {
    const int rc = launch_decode<FMT>(p, stream);
    if (rc) return rc;
  } else {
    const bool pf_ok = p.N % 4 == 0 && p.ldo % 4 == 0 && p.K % kPfBK == 0 &&
                       (reinterpret_cast<uintptr_t>(p.out) & 7) == 0 && block_m <= kPtBM &&
                       (int64_t)kPtBM * p.lda * 2 < 0x7FFFFFFF;
    if (tt && block_m != kPtBM) return -1;   // kernel-argument tables: four-wave kernel only
    if (block_m == kPtBM) {
      // 256-row tiles: the host picks them only where the four-wave kernel
      // takes the shape
      if (!pf_ok || (int64_t)kPtBM * p.ldo * 2 >= 0x7FFFFFFF) return -1;
      const int64_t tiles = (int64_t)p.n_mtiles * ((p.N + kPfBN - 1) / kPfBN);
      // the grid covers eight equal XCD ranges
      const int64_t per_x = prefill_w_per_xcd(tiles, cus);
      if (per_x * 8 > 0x7FFFFFFF) return -1;
      hipLaunchKernelGGL((k_prefill_w<FMT>), dim3((unsigned)(per_x * 8)), dim3(256), 0, stream, p,
                         p.t_row0, p.t_rows, p.t_group, p.eids, p.out, tt ? *tt : no_tiles());
      return hipGetLastError() == hipSuccess ? 0 : -2;
    }
    if (block_m > kPfBM) return -1;
    if (pf_ok) {
      const int64_t tiles = (int64_t)p.n_mtiles * ((p.N + kPfBN - 1) / kPfBN);
      int64_t grid = tiles < cus ? tiles : cus;
      const int dyn = FMT == kNF4 ? 8 * kPairEntries : 0;
      static int configured_dev = -1;
      int dev = 0;
      if (hipGetDevice(&dev) != hipSuccess) return -2;
      if (dyn && configured_dev != dev) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_prefill<FMT, 4>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, dyn) != hipSuccess)
          return -2;
        configured_dev = dev;
      }
      hipLaunchKernelGGL((k_prefill<FMT, 4>), dim3((unsigned)grid), dim3(512), dyn, stream, p,
                         p.t_row0, p.t_rows, p.t_group, p.eids, p.out);
      return hipGetLastError() == hipSuccess ? 0 : -2;
    }
    const int64_t tiles = (int64_t)p.n_mtiles * ((p.N + kBN - 1) / kBN);
    const int64_t grid = clamp_grid(tiles, cus);
    switch (block_m) {
      case 16: hipLaunchKernelGGL((k_gemm_fwd<FMT, 16>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
      case 32: hipLaunchKernelGGL((k_gemm_fwd<FMT, 32>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
      case 64: hipLaunchKernelGGL((k_gemm_fwd<FMT, 64>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
      case 128: hipLaunchKernelGGL((k_gemm_fwd<FMT, 128>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
      default: return -1;
    }
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

template <int FMT>
int launch_dgrad(const DgradArgs& p, int block_m, hipStream_t stream,
                 const PwTiles* tt = nullptr) {
  const int cus = device_cus();
  if (cus <= 0) return -2;
  {
    // the four-wave tile with transposed tr8 reads of the packed rows: any
    // tile of at most 256 rows, whole 64-wide n steps and 64-wide k blocks
    const bool w_ok = p.N % kDgStep == 0 && p.K % 64 == 0 && p.ldo % 4 == 0 &&
                      (reinterpret_cast<uintptr_t>(p.out) & 7) == 0 && block_m <= kPtBM &&
                      (int64_t)kPtBM * p.ldg * 2 < 0x7FFFFFFF &&
                      (int64_t)kPtBM * p.ldo * 2 < 0x7FFFFFFF && p.N * p.sbn < 0x7FFFFFFF &&
                      p.N * p.ssn * 4 < 0x7FFFFFFF;
    if (w_ok) {
      FwdArgs f{};
      f.a = p.g;
      f.lda = p.ldg;
      f.B = p.B;
      f.sbe = p.sbe;
      f.sbn = p.sbn;
      f.S = p.S;
      f.sse = p.sse;
      f.ssn = p.ssn;
      f.n_mtiles = p.n_mtiles;
      f.N = p.N;
      f.K = p.K;
      f.ldo = p.ldo;
      const int64_t tiles = (int64_t)p.n_mtiles * ((p.K + kPfBN - 1) / kPfBN);
      const int64_t per_x = prefill_w_per_xcd(tiles, cus);
      if (per_x * 8 > 0x7FFFFFFF) return -1;
      hipLaunchKernelGGL((k_prefill_w<FMT, true>), dim3((unsigned)(per_x * 8)), dim3(256), 0, stream,
                         f, p.t_row0, p.t_rows, p.t_group, p.eids, p.out, tt ? *tt : no_tiles());
      return hipGetLastError() == hipSuccess ? 0 : -2;
    }
  }
  // a kernel-argument tile table is for the four-wave kernel only: the others
  // read device tables
  if (tt) return -1;
  const bool tiled_ok = p.N % kDgStep == 0 && p.ldo % 4 == 0 &&
                        (reinterpret_cast<uintptr_t>(p.out) & 7) == 0 && block_m <= kPfBM &&
                        (int64_t)kPfBM * p.ldg * 2 < 0x7FFFFFFF && p.N * p.sbn < 0x7FFFFFFF;
  if (block_m > kPfBM) return -1;
  if (tiled_ok) {
    FwdArgs f{};
    f.a = p.g;
    f.lda = p.ldg;
    f.B = p.B;
    f.sbe = p.sbe;
    f.sbn = p.sbn;
    f.S = p.S;
    f.sse = p.sse;
    f.ssn = p.ssn;
    f.n_mtiles = p.n_mtiles;
    f.N = p.N;
    f.K = p.K;
    f.ldo = p.ldo;
    const int64_t tiles = (int64_t)p.n_mtiles * ((p.K + kDgTile - 1) / kDgTile);
    const int64_t grid = tiles < cus ? tiles : cus;
    const int dyn = FMT == kNF4 ? 4 * kPairEntries : 0;   // 16-column table: 32 KiB
    static int configured_dev = -1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -2;
    if (dyn && configured_dev != dev) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_dgrad_tiled<FMT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, dyn) != hipSuccess)
        return -2;
      configured_dev = dev;
    }
    hipLaunchKernelGGL((k_dgrad_tiled<FMT>), dim3((unsigned)grid), dim3(512), dyn, stream, f,
                       p.t_row0, p.t_rows, p.t_group, p.eids, p.out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
  }
  const int64_t tiles = (int64_t)p.n_mtiles * ((p.K + kDgBK - 1) / kDgBK);
  const int64_t grid = clamp_grid(tiles, cus);
  switch (block_m) {
    case 16: hipLaunchKernelGGL((k_gemm_dgrad<FMT, 16>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
    case 32: hipLaunchKernelGGL((k_gemm_dgrad<FMT, 32>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
    case 64: hipLaunchKernelGGL((k_gemm_dgrad<FMT, 64>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
    case 128: hipLaunchKernelGGL((k_gemm_dgrad<FMT, 128>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}


// ----------------------------------------------------- activation widening --
// fp16 / fp32 activations are rounded once to bf16 (nearest-even, the rounding
// torch's .to(bfloat16) applies) so that every forward kernel keeps a single
// bf16 operand type; the bf16 weight path keeps the full fp32 exponent range
// that adversarial absmax values need. One thread converts 8 elements.

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;   // NaN: canonical quiet NaN
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Idx is uint32_t whenever rows * cols / 8 < 2^32: 64-bit division is a long
// software sequence on this GPU.
template <class SrcT, class Idx>
__global__ void __launch_bounds__(256) k_widen_to_bf16(const SrcT* __restrict__ src, int64_t ld_src,
                                                       uint16_t* __restrict__ dst, int64_t ld_dst,
                                                       Idx rows, Idx vec_per_row) {
  const Idx total = rows * vec_per_row;
  for (Idx i = (Idx)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (Idx)gridDim.x * blockDim.x) {
    const int64_t r = i / vec_per_row, c = (i - (Idx)r * vec_per_row) * 8;
    float v[8];
    if constexpr (sizeof(SrcT) == 2) {
      typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
      const f16x8_t h = *reinterpret_cast<const f16x8_t*>(src + r * ld_src + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (float)h[j];
    } else {
      const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(src + r * ld_src + c);
      const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(src + r * ld_src + c + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = lo[j];
        v[4 + j] = hi[j];
      }
    }
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16_rne(v[2 * j]) | (f32_to_bf16_rne(v[2 * j + 1]) << 16);
    *reinterpret_cast<u32x4_t*>(dst + r * ld_dst + c) = o;
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// ------------------------------------------------- no-allocation FFN --
//
// Sync words of gnf4_hip_nf4_ffn_fwd_noalloc: a fixed device array per GPU
// (each device that loads this library holds its own copy until the process
// ends), so that entry point allocates nothing. Zero at load; every call
// that completes leaves its flags zero again. A down unit that times out
// sets word 0 (the sticky error word) and writes NaN, and the gate/up units
// that finish after it leave their flags set to that call's epoch. An eager
// call after that is still exact (it has a new epoch), but a captured graph
// replays its launch with the same epoch, so its next replay could accept
// those flags before its own h is written: after a time-out, run
// gnf4_hip_nf4_ffn_noalloc_reset (stream-ordered, no allocation) before any
// further replay. Calls that overlap on one GPU share the array and race.
constexpr int64_t kFfnScratchWords = int64_t(1) << 19;   // 2 MiB

// Copies word 0 (the error word) to *err (when err is not null) and clears
// all n words: block 0 reads word 0 before its own threads clear it.
__global__ void __launch_bounds__(256) k_ffn_scratch_reset(uint32_t* __restrict__ words, int64_t n,
                                                           uint32_t* __restrict__ err) {
  const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i0 == 0 && err) *err = words[0];
  __syncthreads();
  for (int64_t i = i0; i < n; i += (int64_t)gridDim.x * blockDim.x) words[i] = 0u;
}

}  // namespace

static __device__ __align__(256) uint32_t scratch[kFfnScratchWords];

namespace {

// Device address of `scratch` per device, resolved once with that device
// current (the host-side name is not a device address).
std::mutex g_scratch_mu;
uint32_t* g_scratch_ptr[64] = {};

uint32_t* ffn_scratch_words() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = static_cast<uint32_t*>(ptr);
  }
  return g_scratch_ptr[dev];
}

}  // namespace

namespace {

// Copies host expert ids (and row offsets, when given; else group g is row
// g) into a kernel-argument table, largest groups first (a stable counting
// sort on the row count). 0 on success, -1 on a negative id or decreasing
// offsets, 1 when a group does not fit an entry (more than 255 rows, or a
// first row past kGemvRowsMax): the caller then takes the device tables.
int fill_gemv_ids(GemvIds& gi, const int32_t* expert_ids, const int32_t* row_off, int G) {
  if (G < 1 || G > kGemvIdsMax || !expert_ids) return -1;
  int cnt[kGemvIdsMax], first[kGemvIdsMax];
  for (int g = 0; g < G; ++g) {
    if (expert_ids[g] < 0) return -1;
    if (row_off) {
      if (row_off[g] < 0 || row_off[g + 1] < row_off[g]) return -1;
      cnt[g] = row_off[g + 1] - row_off[g];
      first[g] = row_off[g];
    } else {
      cnt[g] = 1;
      first[g] = g;
    }
  }
  for (int g = 0; g < G; ++g)
    if (cnt[g] > 255 || first[g] >= kGemvRowsMax) return 1;
  // bucket k = 255 - rows: start[k] = how many groups have more rows
  int start[257] = {};
  for (int g = 0; g < G; ++g) ++start[255 - cnt[g] + 1];
  for (int k = 1; k <= 256; ++k) start[k] += start[k - 1];
  for (int g = 0; g < G; ++g) {
    const int y = start[255 - cnt[g]]++;
    gi.e[y] = expert_ids[g];
    gi.rows[y] = first[g] << 8 | cnt[g];
  }
  gi.has_ro = row_off ? 1 : 0;
  gi.n = G;
  return 0;
}

// Checks the fused expert FFN's arguments (all but the id tables and the
// sync words) and fills the two stages' launch arguments; false on bad ones.
bool ffn_stage_args(const void* a, int a_dtype, int64_t lda, const uint8_t* B_gu, int64_t gu_sbe,
                    int64_t gu_sbn, const float* absmax_gu, int64_t gu_sae, int64_t gu_san,
                    const uint8_t* B_dn, int64_t dn_sbe, int64_t dn_sbn, const float* absmax_dn,
                    int64_t dn_sae, int64_t dn_san, bool has_row_off, int G, int max_m,
                    int64_t N_gu, int64_t K, int64_t N_dn, void* h, int64_t ldh, void* out,
                    int64_t ldo, FwdArgs& gu, FwdArgs& dn) {
  if (a_dtype != GNF4_DTYPE_BF16) return false;
  if (N_gu <= 0 || N_gu % 2 || (N_gu / 2) % 64 || K <= 0 || K % 64 || N_dn <= 0 || G < 0)
    return false;
  const int64_t H = N_gu / 2;
  if (max_m < 1 || max_m > 16 || (!has_row_off && max_m != 1)) return false;
  if (!a || !B_gu || !absmax_gu || !B_dn || !absmax_dn || !h || !out) return false;
  if (lda < K || lda % 8 || ldh < H || ldh % 8 || ldo < N_dn || !aligned16(a) || !aligned16(h))
    return false;
  if (gu_sbn % 16 || gu_sbe % 16 || dn_sbn % 16 || dn_sbe % 16 || !aligned16(B_gu) ||
      !aligned16(B_dn))
    return false;
  gu = FwdArgs{};
  gu.a = static_cast<const uint16_t*>(a);
  gu.lda = lda;
  gu.B = B_gu;
  gu.sbe = gu_sbe;
  gu.sbn = gu_sbn;
  gu.S = absmax_gu;
  gu.sse = gu_sae;
  gu.ssn = gu_san;
  gu.G = G;
  gu.max_m = max_m;
  gu.N = N_gu;
  gu.K = K;
  gu.out = static_cast<uint16_t*>(h);
  gu.ldo = ldh;
  dn = gu;
  dn.a = static_cast<const uint16_t*>(h);
  dn.lda = ldh;
  dn.B = B_dn;
  dn.sbe = dn_sbe;
  dn.sbn = dn_sbn;
  dn.S = absmax_dn;
  dn.sse = dn_sae;
  dn.ssn = dn_san;
  dn.N = N_dn;
  dn.K = H;
  dn.out = static_cast<uint16_t*>(out);
  dn.ldo = ldo;
  return true;
}

}  // namespace

// ============================================================== C ABI ====

extern "C" {

int gnf4_hip_abi_version(void) { return GNF4_HIP_ABI_VERSION; }

int gnf4_hip_device_cus(void) { return device_cus(); }

int gnf4_hip_copy_to_device(void* dst, const void* src, int64_t bytes, void* stream) {
  if (bytes < 0 || (bytes > 0 && (!dst || !src))) return -1;
  if (bytes == 0) return 0;
  return hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice,
                        static_cast<hipStream_t>(stream)) == hipSuccess ? 0 : -2;
}

int gnf4_hip_host_device_address(const void* host, void** device) {
  if (!host || !device) return -1;
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, const_cast<void*>(host), 0) != hipSuccess || !d) {
    (void)hipGetLastError();
    return -2;
  }
  *device = d;
  return 0;
}

int gnf4_hip_activations_to_bf16(const void* src, int src_dtype, int64_t rows, int64_t cols,
                                 int64_t ld_src, void* dst, int64_t ld_dst, void* stream) {
  if (src_dtype != GNF4_DTYPE_F16 && src_dtype != GNF4_DTYPE_F32) return -1;
  if (rows < 0 || cols < 0 || cols % 8 || ld_src < cols || ld_dst < cols || ld_src % 8 ||
      ld_dst % 8)
    return -1;
  if (rows == 0 || cols == 0) return 0;
  if (!src || !dst || !aligned16(src) || !aligned16(dst)) return -1;
  const int cus = device_cus();
  if (cus <= 0) return -2;
  const int64_t vec = cols / 8, work = (rows * vec + 255) / 256;
  const int64_t grid = clamp_grid(work, (int64_t)cus * 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool narrow = rows * vec < (int64_t)0xFFFFFFFF;
  if (src_dtype == GNF4_DTYPE_F16 && narrow)
    hipLaunchKernelGGL((k_widen_to_bf16<_Float16, uint32_t>), dim3((unsigned)grid), dim3(256), 0,
                       s, static_cast<const _Float16*>(src), ld_src, static_cast<uint16_t*>(dst),
                       ld_dst, (uint32_t)rows, (uint32_t)vec);
  else if (src_dtype == GNF4_DTYPE_F16)
    hipLaunchKernelGGL((k_widen_to_bf16<_Float16, int64_t>), dim3((unsigned)grid), dim3(256), 0,
                       s, static_cast<const _Float16*>(src), ld_src, static_cast<uint16_t*>(dst),
                       ld_dst, rows, vec);
  else if (narrow)
    hipLaunchKernelGGL((k_widen_to_bf16<float, uint32_t>), dim3((unsigned)grid), dim3(256), 0, s,
                       static_cast<const float*>(src), ld_src, static_cast<uint16_t*>(dst),
                       ld_dst, (uint32_t)rows, (uint32_t)vec);
  else
    hipLaunchKernelGGL((k_widen_to_bf16<float, int64_t>), dim3((unsigned)grid), dim3(256), 0, s,
                       static_cast<const float*>(src), ld_src, static_cast<uint16_t*>(dst),
                       ld_dst, rows, vec);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_silu_mul(const void* gu, int64_t ldg, int64_t T, int64_t H, void* h, int64_t ldh,
                      void* stream) {
  if (T < 0 || H <= 0 || H % 8 || ldg < 2 * H || ldg % 8 || ldh < H || ldh % 8) return -1;
  if (T == 0) return 0;
  if (!gu || !h || !aligned16(gu) || !aligned16(h)) return -1;
  const int cus = device_cus();
  if (cus <= 0) return -2;
  const int64_t work = (T * (H / 8) + 255) / 256;
  const int64_t grid = clamp_grid(work, (int64_t)cus * 8);
  if (T * (H / 8) < (int64_t)0xFFFFFFFF)
    hipLaunchKernelGGL((k_silu_mul<uint32_t>), dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gu), ldg,
                       static_cast<uint16_t*>(h), ldh, (uint32_t)T, (uint32_t)H);
  else
    hipLaunchKernelGGL((k_silu_mul<int64_t>), dim3((unsigned)grid), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gu), ldg,
                       static_cast<uint16_t*>(h), ldh, T, H);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_ffn_set_spin_limit(int polls) {
  if (polls < 0) return -1;
  g_ffn_spin_limit.store(polls, std::memory_order_relaxed);
  return 0;
}

int64_t gnf4_hip_ffn_sync_words(int G, int64_t N_gu, int64_t N_dn) {
  if (G < 0 || N_gu <= 0 || N_dn <= 0) return -1;
  return kFfnFlagBase + (int64_t)G * ((N_dn + 31) / 32) * (N_gu / 32);
}

int gnf4_hip_nf4_ffn_fwd(const void* a, int a_dtype, int64_t lda, const uint8_t* B_gu,
                         int64_t gu_sbe, int64_t gu_sbn, const float* absmax_gu,
                         int64_t gu_sae, int64_t gu_san, const uint8_t* B_dn, int64_t dn_sbe,
                         int64_t dn_sbn, const float* absmax_dn, int64_t dn_sae,
                         int64_t dn_san, const int32_t* expert_ids, const int32_t* row_off,
                         int G, int max_m, int64_t N_gu, int64_t K, int64_t N_dn, void* h,
                         int64_t ldh, uint32_t* sync, int64_t sync_words, void* out,
                         int64_t ldo, void* stream) {
  FwdArgs gu, dn;
  if (!ffn_stage_args(a, a_dtype, lda, B_gu, gu_sbe, gu_sbn, absmax_gu, gu_sae, gu_san, B_dn,
                      dn_sbe, dn_sbn, absmax_dn, dn_sae, dn_san, row_off != nullptr, G, max_m,
                      N_gu, K, N_dn, h, ldh, out, ldo, gu, dn))
    return -1;
  if (!expert_ids || !sync) return -1;
  if (sync_words < gnf4_hip_ffn_sync_words(G, N_gu, N_dn) ||
      ((reinterpret_cast<uintptr_t>(sync) & 3) != 0))
    return -1;
  if (G == 0) return 0;
  const int64_t H = N_gu / 2;
  gu.eids = dn.eids = expert_ids;
  gu.row_off = dn.row_off = row_off;
  if (device_cus() <= 0) return -2;
  const FfnSync fs{sync, next_ffn_epoch(), g_ffn_spin_limit.load(std::memory_order_relaxed)};
  return launch_ffn(gu, dn, H, fs, static_cast<hipStream_t>(stream));
}

int gnf4_hip_nf4_ffn_fwd_noalloc(const void* a, int a_dtype, int64_t lda, const uint8_t* B_gu,
                                 int64_t gu_sbe, int64_t gu_sbn, const float* absmax_gu,
                                 int64_t gu_sae, int64_t gu_san, const uint8_t* B_dn,
                                 int64_t dn_sbe, int64_t dn_sbn, const float* absmax_dn,
                                 int64_t dn_sae, int64_t dn_san, const int32_t* expert_ids,
                                 const int32_t* row_off, int G, int max_m, int64_t N_gu,
                                 int64_t K, int64_t N_dn, void* h, int64_t ldh, void* out,
                                 int64_t ldo, void* stream) {
  const int64_t need = gnf4_hip_ffn_sync_words(G, N_gu, N_dn);
  if (need < 0 || need > kFfnScratchWords) return -1;   // beyond the fixed array
  uint32_t* words = ffn_scratch_words();
  if (!words) return -2;
  return gnf4_hip_nf4_ffn_fwd(a, a_dtype, lda, B_gu, gu_sbe, gu_sbn, absmax_gu, gu_sae, gu_san,
                              B_dn, dn_sbe, dn_sbn, absmax_dn, dn_sae, dn_san, expert_ids,
                              row_off, G, max_m, N_gu, K, N_dn, h, ldh, words,
                              kFfnScratchWords, out, ldo, stream);
}

int gnf4_hip_nf4_ffn_decode_ids(const void* a, int a_dtype, int64_t lda, const uint8_t* B_gu,
                                int64_t gu_sbe, int64_t gu_sbn, const float* absmax_gu,
                                int64_t gu_sae, int64_t gu_san, const uint8_t* B_dn,
                                int64_t dn_sbe, int64_t dn_sbn, const float* absmax_dn,
                                int64_t dn_sae, int64_t dn_san, const int32_t* expert_ids,
                                const int32_t* row_off, int G, int max_m, int64_t N_gu,
                                int64_t K, int64_t N_dn, void* h, int64_t ldh, void* out,
                                int64_t ldo, void* stream) {
  FwdArgs gu, dn;
  if (!ffn_stage_args(a, a_dtype, lda, B_gu, gu_sbe, gu_sbn, absmax_gu, gu_sae, gu_san, B_dn,
                      dn_sbe, dn_sbn, absmax_dn, dn_sae, dn_san, row_off != nullptr, G, max_m,
                      N_gu, K, N_dn, h, ldh, out, ldo, gu, dn))
    return -1;
  if (G == 0) return 0;
  if (!expert_ids) return -1;
  if (G > kGemvIdsMax) return 1;   // the caller takes the device-table entry
  GemvIds gi;
  const int fill = fill_gemv_ids(gi, expert_ids, row_off, G);
  if (fill != 0) return fill;
  const int64_t H = N_gu / 2;
  gu.ids_inline = dn.ids_inline = &gi;
  // both stages must be GEMV launches (the only kernels that read
  // kernel-argument ids): decided before anything is launched
  if (gemv_gu_refuses(gu, H) || gemv_refuses<kNF4>(dn)) return 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int r1 = launch_gemv_gu(gu, H, s);
  if (r1 != 0) return r1 < 0 ? r1 : -2;
  const int r2 = launch_gemv<kNF4>(dn, s);
  return r2 == 0 ? 0 : r2 < 0 ? r2 : -2;
}

int gnf4_hip_nf4_ffn_noalloc_reset(uint32_t* error_word, void* stream) {
  uint32_t* words = ffn_scratch_words();
  if (!words) return -2;
  hipLaunchKernelGGL(k_ffn_scratch_reset, dim3(256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), words, kFfnScratchWords, error_word);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_grouped_fwd(int fmt, const void* a, int a_dtype, int64_t lda, const uint8_t* B,
                         int64_t stride_be, int64_t stride_bn, const void* scales,
                         int64_t stride_se, int64_t stride_sn, const int32_t* expert_ids,
                         const int32_t* row_off, int G, const int32_t* t_row0,
                         const int32_t* t_rows, const int32_t* t_group, int n_mtiles,
                         int block_m, int64_t N, int64_t K, void* out, int64_t ldo,
                         void* stream) {
  const int64_t blk = fmt == GNF4_FMT_NF4 ? 64 : 32;
  if ((fmt != GNF4_FMT_NF4 && fmt != GNF4_FMT_MXFP4) || a_dtype != GNF4_DTYPE_BF16) return -1;
  if (N <= 0 || K <= 0 || K % blk || G < 0 || n_mtiles < 0) return -1;
  if (!a || !B || !scales || !expert_ids || !out) return -1;
  if (lda < K || lda % 8 || ldo < N || stride_bn % 16 || stride_be % 16 || !aligned16(B) ||
      !aligned16(a))
    return -1;
  if (n_mtiles > 0 && (!t_row0 || !t_rows || !t_group)) return -1;
  FwdArgs p{};
  p.a = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = scales;
  p.sse = stride_se;
  p.ssn = stride_sn;
  p.eids = expert_ids;
  p.row_off = row_off;
  p.t_row0 = t_row0;
  p.t_rows = t_rows;
  p.t_group = t_group;
  p.n_mtiles = n_mtiles;
  p.G = G;
  // decode path: block_m carries the largest group size (0: one row each)
  p.max_m = n_mtiles == 0 ? (block_m > 0 ? block_m : 1) : block_m;
  if (n_mtiles == 0 && (p.max_m > 16 || (!row_off && p.max_m != 1))) return -1;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  if (n_mtiles == 0 && G == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return fmt == GNF4_FMT_NF4 ? launch_fwd<kNF4>(p, block_m, s) : launch_fwd<kMX>(p, block_m, s);
}

}  // extern "C"

namespace {
// Host tile tables -> the kernel-argument table; false when they do not fit
// or are inconsistent (ids need a device table unless the tiles carry them).
bool fill_tiles(PwTiles& tt, const int32_t* row0, const int32_t* rows, const int32_t* grp,
                int group_is_expert, int n, const int32_t* expert_ids) {
  if (n <= 0 || n > kPwMaxTiles || !row0 || !rows || !grp) return false;
  if (!group_is_expert && !expert_ids) return false;
  for (int i = 0; i < n; ++i) {
    if (rows[i] <= 0 || rows[i] > kPtBM || row0[i] < 0 || grp[i] < 0) return false;
    tt.row0[i] = row0[i];
    tt.rows[i] = rows[i];
    tt.grp[i] = grp[i];
  }
  tt.n = n;
  tt.grp_is_expert = group_is_expert ? 1 : 0;
  return true;
}
}  // namespace

extern "C" {

int gnf4_hip_grouped_decode_ids(int fmt, const void* a, int a_dtype, int64_t lda,
                                const uint8_t* B, int64_t stride_be, int64_t stride_bn,
                                const void* scales, int64_t stride_se, int64_t stride_sn,
                                const int32_t* expert_ids, const int32_t* row_off, int G,
                                int max_m, int64_t N, int64_t K, void* out, int64_t ldo,
                                void* stream) {
  if (G == 0) return 0;
  if (G < 0 || !expert_ids) return -1;
  if (G > kGemvIdsMax || max_m < 1 || max_m > 16) return 1;   // the caller uploads the tables
  if (max_m > 1 && !row_off) return -1;
  const int64_t blk = fmt == GNF4_FMT_NF4 ? 64 : 32;
  if ((fmt != GNF4_FMT_NF4 && fmt != GNF4_FMT_MXFP4) || a_dtype != GNF4_DTYPE_BF16) return -1;
  if (N <= 0 || K <= 0 || K % blk) return -1;
  if (!a || !B || !scales || !out) return -1;
  if (lda < K || lda % 8 || ldo < N || stride_bn % 16 || stride_be % 16 || !aligned16(B) ||
      !aligned16(a))
    return -1;
  GemvIds gi;
  const int fill = fill_gemv_ids(gi, expert_ids, row_off, G);
  if (fill != 0) return fill;
  FwdArgs p{};
  p.a = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = scales;
  p.sse = stride_se;
  p.ssn = stride_sn;
  p.G = G;
  p.max_m = max_m;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  p.ids_inline = &gi;
  // the tables' pointers stay null: only the GEMV kernels run here, and they
  // read the kernel-argument ids; a launch no GEMV class takes returns 1
  // before anything is launched
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fmt == GNF4_FMT_NF4) {
    if (max_m > 1 && !gemv_nf4_takes_rows(max_m, K)) return 1;
    return launch_gemv<kNF4>(p, s);
  }
  if (max_m > 1) return 1;
  return launch_gemv<kMX>(p, s);
}

int gnf4_hip_grouped_decode_pairs(int fmt, const void* a, int a_dtype, int64_t lda,
                                  const uint8_t* B, int64_t stride_be, int64_t stride_bn,
                                  const void* scales, int64_t stride_se, int64_t stride_sn,
                                  const int32_t* expert_ids, const int32_t* row_pairs, int G,
                                  int max_m, int64_t N, int64_t K, void* out, int64_t ldo,
                                  void* stream) {
  const int64_t blk = fmt == GNF4_FMT_NF4 ? 64 : 32;
  if ((fmt != GNF4_FMT_NF4 && fmt != GNF4_FMT_MXFP4) || a_dtype != GNF4_DTYPE_BF16) return -1;
  if (N <= 0 || K <= 0 || K % blk || G < 0 || max_m < 1 || max_m > 16) return -1;
  if (!a || !B || !scales || !expert_ids || !row_pairs || !out) return -1;
  if (lda < K || lda % 8 || ldo < N || stride_bn % 16 || stride_be % 16 || !aligned16(B) ||
      !aligned16(a))
    return -1;
  if (G == 0) return 0;
  FwdArgs p{};
  p.a = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = scales;
  p.sse = stride_se;
  p.ssn = stride_sn;
  p.eids = expert_ids;
  p.row_off = row_pairs;
  p.ro_shift = 1;
  p.G = G;
  p.max_m = max_m;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return fmt == GNF4_FMT_NF4 ? launch_fwd<kNF4>(p, max_m, s) : launch_fwd<kMX>(p, max_m, s);
}

int gnf4_hip_grouped_decode_routed(int fmt, const void* a, int a_dtype, int64_t lda,
                                   const uint8_t* B, int64_t stride_be, int64_t stride_bn,
                                   const void* scales, int64_t stride_se, int64_t stride_sn,
                                   const int32_t* expert_ids, const int32_t* row_off, int G,
                                   int max_m, int64_t N, int64_t K, void* out, int64_t ldo,
                                   void* stream) {
  const int64_t blk = fmt == GNF4_FMT_NF4 ? 64 : 32;
  if ((fmt != GNF4_FMT_NF4 && fmt != GNF4_FMT_MXFP4) || a_dtype != GNF4_DTYPE_BF16) return -1;
  if (N <= 0 || K <= 0 || K % blk || G < 0 || max_m < 1 || max_m > 16) return -1;
  if (!a || !B || !scales || !expert_ids || !row_off || !out) return -1;
  if (lda < K || lda % 8 || ldo < N || stride_bn % 16 || stride_be % 16 || !aligned16(B) ||
      !aligned16(a))
    return -1;
  if (G == 0) return 0;
  FwdArgs p{};
  p.a = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = scales;
  p.sse = stride_se;
  p.ssn = stride_sn;
  p.eids = expert_ids;
  p.row_off = row_off;
  p.G = G;
  p.max_m = max_m;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  p.sparse_groups = 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return fmt == GNF4_FMT_NF4 ? launch_fwd<kNF4>(p, max_m, s) : launch_fwd<kMX>(p, max_m, s);
}

int gnf4_hip_grouped_fwd_tiles(int fmt, const void* a, int a_dtype, int64_t lda, const uint8_t* B,
                               int64_t stride_be, int64_t stride_bn, const void* scales,
                               int64_t stride_se, int64_t stride_sn, const int32_t* expert_ids,
                               const int32_t* tile_row0, const int32_t* tile_rows,
                               const int32_t* tile_group, int tile_group_is_expert, int n_mtiles,
                               int64_t N, int64_t K, void* out, int64_t ldo, void* stream) {
  if (n_mtiles == 0) return 0;
  if (n_mtiles < 0) return -1;
  if (n_mtiles > kPwMaxTiles) return 1;   // the caller uploads the tables instead
  PwTiles tt;
  if (!fill_tiles(tt, tile_row0, tile_rows, tile_group, tile_group_is_expert, n_mtiles,
                  expert_ids))
    return -1;
  const int64_t blk = fmt == GNF4_FMT_NF4 ? 64 : 32;
  if ((fmt != GNF4_FMT_NF4 && fmt != GNF4_FMT_MXFP4) || a_dtype != GNF4_DTYPE_BF16) return -1;
  if (N <= 0 || K <= 0 || K % blk) return -1;
  if (!a || !B || !scales || !out) return -1;
  if (lda < K || lda % 8 || ldo < N || stride_bn % 16 || stride_be % 16 || !aligned16(B) ||
      !aligned16(a))
    return -1;
  FwdArgs p{};
  p.a = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = scales;
  p.sse = stride_se;
  p.ssn = stride_sn;
  p.eids = expert_ids;
  p.n_mtiles = n_mtiles;
  p.G = 0;
  p.max_m = kPtBM;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return fmt == GNF4_FMT_NF4 ? launch_fwd<kNF4>(p, kPtBM, s, &tt)
                             : launch_fwd<kMX>(p, kPtBM, s, &tt);
}

int gnf4_hip_nf4_fwd(const void* a, int a_dtype, int64_t lda, const uint8_t* B,
                     int64_t stride_be, int64_t stride_bn, const float* absmax,
                     int64_t stride_ae, int64_t stride_an, const int32_t* expert_ids,
                     const int32_t* row_off, int G, const int32_t* t_row0,
                     const int32_t* t_rows, const int32_t* t_group, int n_mtiles, int block_m,
                     int64_t N, int64_t K, void* out, int64_t ldo, void* stream) {
  return gnf4_hip_grouped_fwd(GNF4_FMT_NF4, a, a_dtype, lda, B, stride_be, stride_bn, absmax,
                              stride_ae, stride_an, expert_ids, row_off, G, t_row0, t_rows,
                              t_group, n_mtiles, block_m, N, K, out, ldo, stream);
}

int gnf4_hip_nf4_fwd_fp32w(const void* a, int a_dtype, int64_t lda, const uint8_t* B,
                           int64_t stride_be, int64_t stride_bn, const float* absmax,
                           int64_t stride_ae, int64_t stride_an, const int32_t* expert_ids,
                           const int32_t* t_row0, const int32_t* t_rows, const int32_t* t_group,
                           int n_mtiles, int block_m, int64_t N, int64_t K, void* out,
                           int64_t ldo, void* stream) {
  if (a_dtype != GNF4_DTYPE_BF16 || N <= 0 || K <= 0 || K % 64 || n_mtiles < 0) return -1;
  if (!a || !B || !absmax || !expert_ids || !out) return -1;
  if (lda < K || lda % 8 || ldo < N || stride_bn % 16 || stride_be % 16 || !aligned16(B) ||
      !aligned16(a))
    return -1;
  if (block_m != 16 && block_m != 32 && block_m != 64) return -1;
  if (n_mtiles == 0) return 0;
  if (!t_row0 || !t_rows || !t_group) return -1;
  FwdArgs p{};
  p.a = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = absmax;
  p.sse = stride_ae;
  p.ssn = stride_an;
  p.eids = expert_ids;
  p.t_row0 = t_row0;
  p.t_rows = t_rows;
  p.t_group = t_group;
  p.n_mtiles = n_mtiles;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  const int cus = device_cus();
  if (cus <= 0) return -2;
  const int64_t tiles = (int64_t)n_mtiles * ((N + kBN - 1) / kBN);
  const unsigned grid = (unsigned)clamp_grid(tiles, cus);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (block_m) {
    case 16: hipLaunchKernelGGL((k_gemm_fwd<kNF4, 16, true>), dim3(grid), dim3(kThreads), 0, s, p); break;
    case 32: hipLaunchKernelGGL((k_gemm_fwd<kNF4, 32, true>), dim3(grid), dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((k_gemm_fwd<kNF4, 64, true>), dim3(grid), dim3(kThreads), 0, s, p); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

int gnf4_hip_mxfp4_fwd(const void* a, int a_dtype, int64_t lda, const uint8_t* blocks,
                       int64_t stride_be, int64_t stride_bn, const uint8_t* scales,
                       int64_t stride_se, int64_t stride_sn, const int32_t* expert_ids,
                       const int32_t* row_off, int G, const int32_t* t_row0,
                       const int32_t* t_rows, const int32_t* t_group, int n_mtiles,
                       int block_m, int64_t N, int64_t K, void* out, int64_t ldo,
                       void* stream) {
  return gnf4_hip_grouped_fwd(GNF4_FMT_MXFP4, a, a_dtype, lda, blocks, stride_be, stride_bn,
                              scales, stride_se, stride_sn, expert_ids, row_off, G, t_row0,
                              t_rows, t_group, n_mtiles, block_m, N, K, out, ldo, stream);
}

int gnf4_hip_grouped_dgrad(int fmt, const void* grad_out, int g_dtype, int64_t ldg,
                           const uint8_t* B, int64_t stride_be, int64_t stride_bn,
                           const void* scales, int64_t stride_se, int64_t stride_sn,
                           const int32_t* expert_ids, const int32_t* t_row0,
                           const int32_t* t_rows, const int32_t* t_group, int n_mtiles,
                           int block_m, int64_t N, int64_t K, void* out, int64_t ldo,
                           void* stream) {
  const int64_t blk = fmt == GNF4_FMT_NF4 ? 64 : 32;
  if ((fmt != GNF4_FMT_NF4 && fmt != GNF4_FMT_MXFP4) || g_dtype != GNF4_DTYPE_BF16) return -1;
  if (N <= 0 || K <= 0 || K % blk || n_mtiles < 0) return -1;
  if (!grad_out || !B || !scales || !expert_ids || !out) return -1;
  if (n_mtiles > 0 && (!t_row0 || !t_rows || !t_group)) return -1;
  if (ldg < N || ldg % 8 || ldo < K || stride_bn % 4 || stride_be % 4 || !aligned16(grad_out) ||
      (reinterpret_cast<uintptr_t>(B) & 3))
    return -1;
  if (n_mtiles == 0) return 0;
  DgradArgs p;
  p.g = static_cast<const uint16_t*>(grad_out);
  p.ldg = ldg;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = scales;
  p.sse = stride_se;
  p.ssn = stride_sn;
  p.eids = expert_ids;
  p.t_row0 = t_row0;
  p.t_rows = t_rows;
  p.t_group = t_group;
  p.n_mtiles = n_mtiles;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return fmt == GNF4_FMT_NF4 ? launch_dgrad<kNF4>(p, block_m, s)
                             : launch_dgrad<kMX>(p, block_m, s);
}

int gnf4_hip_grouped_dgrad_tiles(int fmt, const void* grad_out, int g_dtype, int64_t ldg,
                                 const uint8_t* B, int64_t stride_be, int64_t stride_bn,
                                 const void* scales, int64_t stride_se, int64_t stride_sn,
                                 const int32_t* expert_ids, const int32_t* tile_row0,
                                 const int32_t* tile_rows, const int32_t* tile_group,
                                 int tile_group_is_expert, int n_mtiles, int64_t N, int64_t K,
                                 void* out, int64_t ldo, void* stream) {
  if (n_mtiles == 0) return 0;
  if (n_mtiles < 0) return -1;
  if (n_mtiles > kPwMaxTiles) return 1;   // the caller uploads the tables instead
  PwTiles tt;
  if (!fill_tiles(tt, tile_row0, tile_rows, tile_group, tile_group_is_expert, n_mtiles,
                  expert_ids))
    return -1;
  const int64_t blk = fmt == GNF4_FMT_NF4 ? 64 : 32;
  if ((fmt != GNF4_FMT_NF4 && fmt != GNF4_FMT_MXFP4) || g_dtype != GNF4_DTYPE_BF16) return -1;
  if (N <= 0 || K <= 0 || K % blk) return -1;
  if (!grad_out || !B || !scales || !out) return -1;
  if (ldg < N || ldg % 8 || ldo < K || stride_bn % 4 || stride_be % 4 || !aligned16(grad_out) ||
      (reinterpret_cast<uintptr_t>(B) & 3))
    return -1;
  DgradArgs p;
  p.g = static_cast<const uint16_t*>(grad_out);
  p.ldg = ldg;
  p.B = B;
  p.sbe = stride_be;
  p.sbn = stride_bn;
  p.S = scales;
  p.sse = stride_se;
  p.ssn = stride_sn;
  p.eids = expert_ids;
  p.t_row0 = nullptr;
  p.t_rows = nullptr;
  p.t_group = nullptr;
  p.n_mtiles = n_mtiles;
  p.N = N;
  p.K = K;
  p.out = static_cast<uint16_t*>(out);
  p.ldo = ldo;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return fmt == GNF4_FMT_NF4 ? launch_dgrad<kNF4>(p, kPtBM, s, &tt)
                             : launch_dgrad<kMX>(p, kPtBM, s, &tt);
}

int gnf4_hip_nf4_dgrad(const void* grad_out, int g_dtype, int64_t ldg, const uint8_t* B,
                       int64_t stride_be, int64_t stride_bn, const float* absmax,
                       int64_t stride_ae, int64_t stride_an, const int32_t* expert_ids,
                       const int32_t* t_row0, const int32_t* t_rows, const int32_t* t_group,
                       int n_mtiles, int block_m, int64_t N, int64_t K, void* out, int64_t ldo,
                       void* stream) {
  return gnf4_hip_grouped_dgrad(GNF4_FMT_NF4, grad_out, g_dtype, ldg, B, stride_be, stride_bn,
                                absmax, stride_ae, stride_an, expert_ids, t_row0, t_rows,
                                t_group, n_mtiles, block_m, N, K, out, ldo, stream);
}

int gnf4_hip_mxfp4_dgrad(const void* grad_out, int g_dtype, int64_t ldg, const uint8_t* blocks,
                         int64_t stride_be, int64_t stride_bn, const uint8_t* scales,
                         int64_t stride_se, int64_t stride_sn, const int32_t* expert_ids,
                         const int32_t* t_row0, const int32_t* t_rows, const int32_t* t_group,
                         int n_mtiles, int block_m, int64_t N, int64_t K, void* out,
                         int64_t ldo, void* stream) {
  return gnf4_hip_grouped_dgrad(GNF4_FMT_MXFP4, grad_out, g_dtype, ldg, blocks, stride_be,
                                stride_bn, scales, stride_se, stride_sn, expert_ids, t_row0,
                                t_rows, t_group, n_mtiles, block_m, N, K, out, ldo, stream);
}

}  // extern "C"
