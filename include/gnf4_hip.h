/* gnf4_hip.h -- C ABI of libgnf4_hip.so, the grouped 4-bit MoE expert GEMM
 * for AMD Instinct MI355X (gfx950).
 *
 * Plain pointers and sizes only. All pointers are device pointers except
 * `stream`, which is a hipStream_t (pass torch.cuda.current_stream().cuda_stream).
 * The group tables of a decode-path launch (expert_ids, row_off) may also
 * be pinned host memory at its device address (gnf4_hip_host_device_address):
 * each workgroup reads its group's words once. Tile tables should be device
 * memory: the tiled kernels read them once per tile.
 * Every call is asynchronous and stream-ordered; none allocates or synchronises.
 *
 * Shared conventions (reference docs/KERNEL_CONTRACT.md, kernel/nf4_grouped.py:697-725):
 *   a / grad_out  [T, ld] bf16 (a_dtype / g_dtype GNF4_DTYPE_BF16; fp16
 *                 and fp32 activations go through
 *                 gnf4_hip_activations_to_bf16 first), rows sorted by group (group g owns rows
 *                 row_off[g] .. row_off[g+1]); ld % 8 == 0, 16-byte aligned.
 *   B / blocks    [E, N, K/2] uint8, last dimension contiguous; strides in
 *                 BYTES, multiples of 16 (forward) / 4 (dgrad).
 *   absmax        [E, N, K/64] fp32 (NF4, K % 64 == 0), strides in elements.
 *   scales        [E, N, K/32] uint8 e8m0 (MXFP4, K % 32 == 0), strides in elements.
 *   expert_ids    [G] int32: expert of group g.
 *   out           [T, ldo] bf16.
 * Offsets into B are formed in 64-bit arithmetic (stacks above 2^31 bytes,
 * reference kernel/nf4_grouped.py:396-399).
 *
 * Path selection (forward):
 *   n_mtiles == 0 -> decode path: every group holds <= 16 rows (the caller
 *                    guarantees it); `row_off` [G + 1] int32 gives each
 *                    group's rows, or is NULL when every group is exactly
 *                    one row (group g is row g, as in the reference's
 *                    decode grid); the tile table is ignored and block_m
 *                    carries the largest group size (0 or 1 with a NULL
 *                    row_off; at most 16).
 *   n_mtiles  > 0 -> tiled path: the tile table t_row0/t_rows/t_group
 *                    [n_mtiles] int32 (reference build_group_tiles,
 *                    kernel/nf4_grouped.py:334-362) with block_m in
 *                    {16, 32, 64, 128, 256}; t_rows[i] <= block_m. 256
 *                    selects the four-wave tall-tile kernel and needs
 *                    K % 64 == 0, N % 4 == 0, ldo % 4 == 0 and an 8-byte
 *                    aligned out (-1 otherwise). The tile order is free
 *                    (each XCD takes a contiguous eighth of the list).
 *
 * Return codes (the reference CPU tier's convention, gnf4_native/cpu_kernels.c:745-761):
 *   0 success, -1 shape or argument violation, -2 launch error.
 */
#ifndef GNF4_HIP_H_
#define GNF4_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GNF4_HIP_ABI_VERSION 14

#define GNF4_FMT_NF4 0
#define GNF4_FMT_MXFP4 1

#define GNF4_DTYPE_BF16 0
#define GNF4_DTYPE_F16 1
#define GNF4_DTYPE_F32 2

/* ABI version of the loaded library (GNF4_HIP_ABI_VERSION). */
int gnf4_hip_abi_version(void);

/* Compute units of the current device (0 on error). Replaces the reference's
 * torch-side SM query `_sm_count` (kernel/nf4_grouped.py:581-591). */
int gnf4_hip_device_cus(void);

/* Stream-ordered copy of `bytes` bytes of pinned host memory to device memory
 * (hipMemcpyAsync on `stream`): the upload of one call's group tables (expert
 * ids, row offsets, tile table) into a device staging ring, without a torch
 * tensor per call. The reference uploads the same tables with a torch copy
 * (to_device_i32, kernel/nf4_grouped.py:229-331). The host bytes must stay
 * unchanged until the copy has run. 0 on success, -1 on bad arguments, -2 on
 * a runtime error. */
int gnf4_hip_copy_to_device(void *dst, const void *src, int64_t bytes, void *stream);

/* The device address of pinned host memory (hipHostGetDevicePointer): decode
 * launches read their group tables (expert ids, row offsets) straight from a
 * pinned host ring at this address, with no copy; each workgroup reads its
 * group's three words once. The reference uploads the same tables with a
 * torch copy (to_device_i32, kernel/nf4_grouped.py:229-331). 0 on success,
 * -1 on bad arguments, -2 when the memory is not mapped for the current
 * device. */
int gnf4_hip_host_device_address(const void *host, void **device);

/* Round fp16 (src_dtype GNF4_DTYPE_F16) or fp32 (GNF4_DTYPE_F32) activations
 * [rows, ld_src] to bf16 [rows, ld_dst], nearest-even (NaN -> 0x7FC0), so a
 * forward call can take them. The reference's kernels accept fp16 and fp32
 * activations and widen them in-register (kernel/nf4_grouped.py:456-458,
 * 511; kernel/mxfp4_grouped.py:94; docs/KERNEL_CONTRACT.md:25); here one
 * bf16 operand type keeps the weights in bf16's fp32-wide exponent range.
 * cols, ld_src and ld_dst multiples of 8; src and dst 16-byte aligned. */
int gnf4_hip_activations_to_bf16(const void *src, int src_dtype, int64_t rows,
                                 int64_t cols, int64_t ld_src, void *dst,
                                 int64_t ld_dst, void *stream);

/* Grouped forward for either format: out[t, :] = a[t, :] . dequant(W[e(t)])^T,
 * fp32 accumulation, one bf16 rounding per output. Replaces the launches in
 * gemm_4bit_grouped (reference kernel/nf4_grouped.py:750-906: the
 * _gemv_nf4_grouped / _gemv_nf4_grouped_splitk / _gemm_nf4_grouped grids) and
 * gemm_mxfp4_grouped (kernel/mxfp4_grouped.py:146-171). */
int gnf4_hip_grouped_fwd(int fmt, const void *a, int a_dtype, int64_t lda,
                         const uint8_t *B, int64_t stride_be, int64_t stride_bn,
                         const void *scales, int64_t stride_se, int64_t stride_sn,
                         const int32_t *expert_ids, const int32_t *row_off, int G,
                         const int32_t *t_row0, const int32_t *t_rows,
                         const int32_t *t_group, int n_mtiles, int block_m,
                         int64_t N, int64_t K, void *out, int64_t ldo, void *stream);

/* Grouped decode forward with the expert ids (and row offsets) in host
 * memory, for launches of at most 384 groups in a GEMV class: groups of one
 * row (NF4 and MXFP4), or NF4 groups of up to 4 rows at 1024 < K <= 2048 (2
 * rows at K <= 1024). The ids travel in the kernel's arguments, so the
 * kernel reads no table before its first weight load, the call makes no
 * upload, and a captured call is the kernel node alone. Same bits as
 * gnf4_hip_grouped_fwd's decode path with the same ids. expert_ids[G] and
 * row_off[G + 1] (NULL: group g is row g, max_m = 1) are read before the
 * call returns. The kernel's grid takes the groups largest first (the
 * workgroups that make the most passes start first; no bits change).
 * Returns 1, launching nothing, when G > 384, a group has more than 255
 * rows or starts past row 2^23, or no GEMV class takes the launch (the
 * caller then uploads the tables and calls gnf4_hip_grouped_fwd). Replaces the decode launches of gemm_4bit_grouped /
 * gemm_mxfp4_grouped, reference kernel/nf4_grouped.py:750-806,
 * kernel/mxfp4_grouped.py:146-160 (whose expert ids go through
 * to_device_i32, kernel/nf4_grouped.py:229-331). */
int gnf4_hip_grouped_decode_ids(int fmt, const void *a, int a_dtype, int64_t lda,
                                const uint8_t *B, int64_t stride_be, int64_t stride_bn,
                                const void *scales, int64_t stride_se, int64_t stride_sn,
                                const int32_t *expert_ids, const int32_t *row_off, int G,
                                int max_m, int64_t N, int64_t K, void *out, int64_t ldo,
                                void *stream);

/* Grouped decode forward (every group at most max_m <= 16 rows) whose row
 * table is a (first row, end row) pair per group, row_pairs[2 G] in device
 * memory (or pinned host memory at its device address), next to
 * expert_ids[G]: group g covers rows [row_pairs[2 g], row_pairs[2 g + 1]).
 * The groups need not come in row order, so a caller can list them largest
 * first, and the workgroups of the groups with the most rows are
 * dispatched first. Same kernels and bits per row as gnf4_hip_grouped_fwd's
 * decode path. Returns -1 on bad arguments (as gnf4_hip_grouped_fwd). No
 * counterpart in the reference; it replaces the decode launches of
 * gemm_4bit_grouped / gemm_mxfp4_grouped (reference
 * kernel/nf4_grouped.py:750-806, kernel/mxfp4_grouped.py:146-160) for
 * callers that hold the group sizes on the host. */
int gnf4_hip_grouped_decode_pairs(int fmt, const void *a, int a_dtype, int64_t lda,
                                  const uint8_t *B, int64_t stride_be, int64_t stride_bn,
                                  const void *scales, int64_t stride_se, int64_t stride_sn,
                                  const int32_t *expert_ids, const int32_t *row_pairs, int G,
                                  int max_m, int64_t N, int64_t K, void *out, int64_t ldo,
                                  void *stream);

/* Grouped decode forward over device-routing tables (gnf4_hip_route_groups
 * / gnf4_hip_route_decode: eids [G], row_off [G + 1], G = their slots, max_m
 * a bound of the largest group), where any group may be empty: the same
 * kernels and bits as gnf4_hip_grouped_fwd's decode path, minus the unit
 * walk that deals its workgroups to the groups in equal shares (the shares
 * of empty groups would idle). -1 on bad arguments. No counterpart in the
 * reference (its routing is on the host, kernel/arena_moe_patch.py:41-66). */
int gnf4_hip_grouped_decode_routed(int fmt, const void *a, int a_dtype, int64_t lda,
                                   const uint8_t *B, int64_t stride_be, int64_t stride_bn,
                                   const void *scales, int64_t stride_se, int64_t stride_sn,
                                   const int32_t *expert_ids, const int32_t *row_off, int G,
                                   int max_m, int64_t N, int64_t K, void *out, int64_t ldo,
                                   void *stream);

/* Grouped forward on 256-row tiles with the tile table in host memory: the
 * table (at most 256 m-tiles) travels in the kernel's arguments, so the call
 * makes no copy ahead of its launch and a captured graph holds the kernel
 * node alone. Same computation and bits as gnf4_hip_grouped_fwd with
 * block_m = 256 and the same table. tile_row0 / tile_rows / tile_group are
 * host arrays of n_mtiles int32, read before the call returns. With
 * tile_group_is_expert = 1, tile_group holds each tile's expert id and
 * expert_ids may be NULL; otherwise it holds group indices into the device
 * array expert_ids. Returns 1, launching nothing, when n_mtiles > 256 (the
 * caller uploads the table and calls gnf4_hip_grouped_fwd), -1 on a shape
 * the 256-row kernel does not take or an inconsistent table. Replaces the
 * same launch as gnf4_hip_grouped_fwd, reference
 * kernel/nf4_grouped.py:750-906 (its tile tables go through
 * to_device_i32, :229-331). */
int gnf4_hip_grouped_fwd_tiles(int fmt, const void *a, int a_dtype, int64_t lda,
                               const uint8_t *B, int64_t stride_be, int64_t stride_bn,
                               const void *scales, int64_t stride_se, int64_t stride_sn,
                               const int32_t *expert_ids, const int32_t *tile_row0,
                               const int32_t *tile_rows, const int32_t *tile_group,
                               int tile_group_is_expert, int n_mtiles, int64_t N, int64_t K,
                               void *out, int64_t ldo, void *stream);

/* NF4 forward (absmax fp32, block 64). Replaces the NF4 kernel launches of
 * gemm_4bit_grouped, reference kernel/nf4_grouped.py:750-906. */
int gnf4_hip_nf4_fwd(const void *a, int a_dtype, int64_t lda, const uint8_t *B,
                     int64_t stride_be, int64_t stride_bn, const float *absmax,
                     int64_t stride_ae, int64_t stride_an, const int32_t *expert_ids,
                     const int32_t *row_off, int G, const int32_t *t_row0,
                     const int32_t *t_rows, const int32_t *t_group, int n_mtiles,
                     int block_m, int64_t N, int64_t K, void *out, int64_t ldo,
                     void *stream);

/* NF4 tiled forward with fp32-precision weights: the reference's default
 * M-tile numerics (VARIANT 1, kernel/nf4_grouped.py:446-452: fp32 decoded
 * weights LUT x absmax in the dot), selected there by prefill_variant=1.
 * Each weight w = LUT[code] * absmax (fp32, one rounding) enters the bf16
 * MFMA as hi = bf16(w) plus lo = bf16(w - hi), two MFMAs per k-slice, so the
 * products carry w to within 2^-17 of |w| (the default tiled kernels round
 * w to bf16 once). Tile table as for gnf4_hip_nf4_fwd's tiled path, with
 * block_m in {16, 32, 64} (t_rows[i] <= block_m). Costs about twice the
 * matrix work of the default tiles on a simpler kernel. 0 / -1 / -2. */
int gnf4_hip_nf4_fwd_fp32w(const void *a, int a_dtype, int64_t lda, const uint8_t *B,
                           int64_t stride_be, int64_t stride_bn, const float *absmax,
                           int64_t stride_ae, int64_t stride_an, const int32_t *expert_ids,
                           const int32_t *t_row0, const int32_t *t_rows,
                           const int32_t *t_group, int n_mtiles, int block_m, int64_t N,
                           int64_t K, void *out, int64_t ldo, void *stream);

/* MXFP4 forward (e2m1 nibbles, e8m0 scale per 32). Replaces the launches of
 * gemm_mxfp4_grouped, reference kernel/mxfp4_grouped.py:146-171. */
int gnf4_hip_mxfp4_fwd(const void *a, int a_dtype, int64_t lda, const uint8_t *blocks,
                       int64_t stride_be, int64_t stride_bn, const uint8_t *scales,
                       int64_t stride_se, int64_t stride_sn, const int32_t *expert_ids,
                       const int32_t *row_off, int G, const int32_t *t_row0,
                       const int32_t *t_rows, const int32_t *t_group, int n_mtiles,
                       int block_m, int64_t N, int64_t K, void *out, int64_t ldo,
                       void *stream);

/* Elementwise gate activation of the expert FFN, unfused form:
 *   h[t, j] = bf16(silu_locked(gu[t, j]) * gu[t, H + j]),  j < H,
 * gu [T, ldg] bf16 (gate = first H columns, up = next H), h [T, ldh] bf16.
 * silu_locked is the reference's fixed fp32 op sequence
 * (gnf4_native/cpu_kernels.c:776-822, kernel/cpu_grouped.py:147-179):
 * clamp at +-87 with exact tails, degree-6 Horner 2^f, 1 / (1 + e), no FMA.
 * H, ldg, ldh multiples of 8; gu and h 16-byte aligned. */
int gnf4_hip_silu_mul(const void *gu, int64_t ldg, int64_t T, int64_t H, void *h,
                      int64_t ldh, void *stream);

/* Fused NF4 expert FFN at decode, one call: out = dn(silu(gate) * up) with
 * gate/up the two halves of a . W_gu^T. Groups of one row run two launches
 * (the gate_up GEMV with the silu-multiply in its epilogue, then the down
 * GEMV; `sync` unused); larger groups one launch whose down units wait for
 * h through the sync flags. Same bits as gate_up forward -> silu-multiply ->
 * down forward either way. GPU counterpart of the reference's
 * CPU gnf4_gemv_nf4_ffn_grouped (gnf4_native/cpu_kernels.c:948-986, spec
 * kernel/cpu_grouped.py:182-194), which has no GPU kernel there.
 *   a     [T, lda] bf16, rows sorted by group; every group <= 16 rows
 *         (max_m = the largest, 1..16; row_off [G + 1] as for the decode
 *         forward, NULL only when every group is one row).
 *   W_gu  [E, N_gu, K/2] u8 + absmax [E, N_gu, K/64] f32, H = N_gu / 2,
 *         H % 64 == 0, K % 64 == 0.
 *   W_dn  [E, N_dn, H/2] u8 + absmax [E, N_dn, H/64] f32.
 *   h     [T, ldh] bf16 workspace (the intermediate; ldh >= H, % 8 == 0).
 *   sync  >= gnf4_hip_ffn_sync_words(G, N_gu, N_dn) u32 words, zero
 *         before the first call; every call leaves its flags zero again
 *         (graph replays included). Calls that overlap on one sync buffer
 *         race. Word 0 is a sticky error flag: it becomes nonzero if a down
 *         unit gave up waiting for h (never expected), and that unit's
 *         output rows are NaN. Flags carry a per-call epoch, so flags left
 *         behind by such a call are never taken for a later call's; graph
 *         replays reuse the epoch captured with them, so after an error a
 *         replayed graph's result is invalid until the caller clears the
 *         sync buffer.
 *   out   [T, ldo] bf16.
 * h is bf16(silu_locked(bf16(gate)) * bf16(up)), so the result equals
 * gnf4_hip_nf4_fwd (gate_up) -> gnf4_hip_silu_mul -> gnf4_hip_nf4_fwd (down)
 * bit for bit. */
/* Size (u32 words) of the sync buffer gnf4_hip_nf4_ffn_fwd needs for G
 * groups: one flag per (gate/up unit, down unit) pair of a group, plus a
 * header. -1 on bad arguments. No counterpart in the reference (its fused
 * FFN is CPU-only). */
int64_t gnf4_hip_ffn_sync_words(int G, int64_t N_gu, int64_t N_dn);

/* Polls a fused-FFN down unit makes before it gives up waiting for h
 * (default 2^22), for launches after this call. A diagnostics and test
 * knob: 0 makes every down unit that does not find its h ready at the first
 * poll write NaN and set the error word. -1 on a negative value. No
 * counterpart in the reference. */
int gnf4_hip_ffn_set_spin_limit(int polls);

int gnf4_hip_nf4_ffn_fwd(const void *a, int a_dtype, int64_t lda, const uint8_t *B_gu,
                         int64_t gu_sbe, int64_t gu_sbn, const float *absmax_gu,
                         int64_t gu_sae, int64_t gu_san, const uint8_t *B_dn,
                         int64_t dn_sbe, int64_t dn_sbn, const float *absmax_dn,
                         int64_t dn_sae, int64_t dn_san, const int32_t *expert_ids,
                         const int32_t *row_off, int G, int max_m, int64_t N_gu, int64_t K,
                         int64_t N_dn, void *h, int64_t ldh, uint32_t *sync,
                         int64_t sync_words, void *out, int64_t ldo, void *stream);

/* gnf4_hip_nf4_ffn_fwd without the sync argument, for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * sync words live in a fixed per-GPU array of the library (2 MiB, held
 * until the process ends); the call allocates nothing. Returns -1 when
 * gnf4_hip_ffn_sync_words(G, N_gu, N_dn) exceeds 524288 words (the
 * array's size), otherwise what gnf4_hip_nf4_ffn_fwd returns. Every call on
 * a GPU shares that GPU's array: calls that overlap on one GPU race (run
 * them in one stream order). A down unit that times out writes NaN into
 * its output rows and sets the array's error word; read and clear it with
 * gnf4_hip_nf4_ffn_noalloc_reset. Under graph capture the call's epoch is
 * fixed in the graph: after a replay that timed out, run the reset before
 * replaying again (otherwise flags left by that replay's late gate/up units
 * could pass the next replay's down units early). */
int gnf4_hip_nf4_ffn_fwd_noalloc(const void *a, int a_dtype, int64_t lda,
                                 const uint8_t *B_gu, int64_t gu_sbe, int64_t gu_sbn,
                                 const float *absmax_gu, int64_t gu_sae, int64_t gu_san,
                                 const uint8_t *B_dn, int64_t dn_sbe, int64_t dn_sbn,
                                 const float *absmax_dn, int64_t dn_sae, int64_t dn_san,
                                 const int32_t *expert_ids, const int32_t *row_off, int G,
                                 int max_m, int64_t N_gu, int64_t K, int64_t N_dn, void *h,
                                 int64_t ldh, void *out, int64_t ldo, void *stream);

/* gnf4_hip_nf4_ffn_fwd with host group tables: expert_ids [G] and row_off
 * [G + 1] (NULL when every group is one row) are host int32 arrays, copied
 * into the kernels' arguments, so nothing is uploaded and the kernels read
 * no table ahead of the weights. Runs only when both stages are GEMV
 * launches (groups of one row; or, with row_off, groups of at most 4 rows
 * at 1024 < K <= 2048 and 2 at K <= 1024 for each stage's K) and
 * G <= 384; otherwise returns 1 before launching anything and the caller
 * takes gnf4_hip_nf4_ffn_fwd. Same bits as gnf4_hip_nf4_ffn_fwd; no sync
 * words. Same operation as the reference's CPU gnf4_gemv_nf4_ffn_grouped
 * (gnf4_native/cpu_kernels.c:948-986), whose ids are host arrays too. 0 on
 * success, -1 on bad arguments (a negative id, decreasing offsets), -2 on a
 * runtime error. */
int gnf4_hip_nf4_ffn_decode_ids(const void *a, int a_dtype, int64_t lda, const uint8_t *B_gu,
                                int64_t gu_sbe, int64_t gu_sbn, const float *absmax_gu,
                                int64_t gu_sae, int64_t gu_san, const uint8_t *B_dn,
                                int64_t dn_sbe, int64_t dn_sbn, const float *absmax_dn,
                                int64_t dn_sae, int64_t dn_san, const int32_t *expert_ids,
                                const int32_t *row_off, int G, int max_m, int64_t N_gu,
                                int64_t K, int64_t N_dn, void *h, int64_t ldh, void *out,
                                int64_t ldo, void *stream);

/* Stream-ordered read and clear of the fixed sync array of
 * gnf4_hip_nf4_ffn_fwd_noalloc on the current device: copies its error word
 * (nonzero when a down unit of an earlier call timed out) to *error_word
 * (device memory, or pinned host memory at its device address; may be
 * NULL), then zeroes the whole array with a kernel (no hipMemsetAsync, so
 * it can be captured in a graph). Allocates nothing. No counterpart in the
 * reference; for the same callers as the no-allocation entry point. 0 on
 * success, -2 on a runtime error. */
int gnf4_hip_nf4_ffn_noalloc_reset(uint32_t *error_word, void *stream);

/* Grouped dgrad for either format: out[t, :] = grad_out[t, :] . dequant(W[e(t)]),
 * contracting over N in fixed 64-wide ascending steps (output bits do not
 * depend on block_m). grad_out is [T, ldg] bf16, out is [T, ldo] bf16 with
 * ldo >= K. Tile table as for the forward tiled path (n_mtiles may be 0:
 * nothing to do). With N % 64 == 0 and K % 64 == 0 any block_m up to 256
 * runs the four-wave transposed-read kernel; other shapes need
 * block_m <= 128 (-1 otherwise). */
int gnf4_hip_grouped_dgrad(int fmt, const void *grad_out, int g_dtype, int64_t ldg,
                           const uint8_t *B, int64_t stride_be, int64_t stride_bn,
                           const void *scales, int64_t stride_se, int64_t stride_sn,
                           const int32_t *expert_ids, const int32_t *t_row0,
                           const int32_t *t_rows, const int32_t *t_group, int n_mtiles,
                           int block_m, int64_t N, int64_t K, void *out, int64_t ldo,
                           void *stream);

/* Grouped dgrad on 256-row tiles with the tile table in host memory, in the
 * kernel's arguments (as gnf4_hip_grouped_fwd_tiles): same bits as
 * gnf4_hip_grouped_dgrad with the same table. Needs N % 64 == 0 and
 * K % 64 == 0 (-1 otherwise); returns 1 without launching when
 * n_mtiles > 256. Replaces the launch of dgrad_4bit_grouped, reference
 * kernel/nf4_grouped.py:1100-1120. */
int gnf4_hip_grouped_dgrad_tiles(int fmt, const void *grad_out, int g_dtype, int64_t ldg,
                                 const uint8_t *B, int64_t stride_be, int64_t stride_bn,
                                 const void *scales, int64_t stride_se, int64_t stride_sn,
                                 const int32_t *expert_ids, const int32_t *tile_row0,
                                 const int32_t *tile_rows, const int32_t *tile_group,
                                 int tile_group_is_expert, int n_mtiles, int64_t N, int64_t K,
                                 void *out, int64_t ldo, void *stream);

/* NF4 dgrad. Replaces the _dgrad_nf4_grouped launch of dgrad_4bit_grouped,
 * reference kernel/nf4_grouped.py:1100-1120. */
int gnf4_hip_nf4_dgrad(const void *grad_out, int g_dtype, int64_t ldg, const uint8_t *B,
                       int64_t stride_be, int64_t stride_bn, const float *absmax,
                       int64_t stride_ae, int64_t stride_an, const int32_t *expert_ids,
                       const int32_t *t_row0, const int32_t *t_rows,
                       const int32_t *t_group, int n_mtiles, int block_m, int64_t N,
                       int64_t K, void *out, int64_t ldo, void *stream);

/* MXFP4 dgrad. The reference has no GPU kernel for it (its backward is a
 * per-expert Python loop, kernel/mxfp4_qlora.py:106-122); the CPU spec it
 * follows is gnf4_dgrad_mxfp4_grouped, gnf4_native/cpu_kernels.c:1386-1397. */
int gnf4_hip_mxfp4_dgrad(const void *grad_out, int g_dtype, int64_t ldg,
                         const uint8_t *blocks, int64_t stride_be, int64_t stride_bn,
                         const uint8_t *scales, int64_t stride_se, int64_t stride_sn,
                         const int32_t *expert_ids, const int32_t *t_row0,
                         const int32_t *t_rows, const int32_t *t_group, int n_mtiles,
                         int block_m, int64_t N, int64_t K, void *out, int64_t ldo,
                         void *stream);

/* ---------------------------------------------------------- routing --
 * Device-side routing around the grouped GEMM, so a decode MoE layer needs
 * no host read of the routing and can be captured in one graph. */

/* Top-k selection with softmax weights, one token per row of logits
 * [T, ld] fp32: idx [T, idx_stride] int64 and wts [T, wts_stride] bf16 bits.
 * GPU counterpart of gnf4_route_epilogue_bf16 (reference
 * gnf4_native/cpu_kernels.c:1408-1471), same arguments plus ld and stream:
 * selection in stable-descending order (ties to the lower index); mode 0 =
 * softmax over all E logits gathered at the selection, renormalised over it
 * when norm != 0 (olmoe/qwen3); mode 1 = softmax over the k selected logits
 * (gpt_oss). k <= 64 and k <= E <= 1024. NaN logits: unspecified. */
int gnf4_hip_route_topk(const float *logits, int64_t T, int64_t E, int64_t ld, int k,
                        int mode, int norm, int64_t *idx, int64_t idx_stride,
                        uint16_t *wts, int64_t wts_stride, void *stream);

/* Groups the N = T * k rows (row i = token i / k, slot i % k) of topk_ids
 * [T, ids_stride] int64 by expert: the sort / count of the reference's MoE
 * dispatch (kernel/arena_moe_patch.py:41-47), on the device. Active experts
 * become groups in ascending expert order; rows of one expert keep row
 * order. Writes eids [slots] int32, row_off [slots + 1] int32 (groups past
 * the active count are empty), order [N] int32 (grouped position -> row),
 * pos [N] int32 (row -> grouped position, -1 for an id outside [0, E)),
 * info [3] int32 (active groups, largest group, 1 if an id was out of
 * range). E <= 512. cap > 0 splits an expert's rows into consecutive
 * groups of at most cap rows (same expert id; cap = 0: one group per
 * expert), so the largest group is at most cap rows and a decode launch
 * can take the class of cap rows instead of T. With M = min(N, E), slots =
 * M + (N - M) / cap (slots = M when cap = 0) holds every case; the tables
 * can be passed straight to the decode forward / fused FFN with G = slots.
 * (The reference's dispatch has one group per expert; the split groups
 * give every row the bits of the same rows in one group of that class.) */
int gnf4_hip_route_groups(const int64_t *topk_ids, int64_t ids_stride, int64_t T, int k,
                          int64_t E, int slots, int cap, int32_t *eids, int32_t *row_off,
                          int32_t *order, int32_t *pos, int32_t *info, void *stream);

/* The decode routing prologue in one launch (T <= 16 tokens, E <= 512):
 * gnf4_hip_route_topk (skipped when logits is NULL: idx then holds the
 * caller's ids), gnf4_hip_route_groups and gnf4_hip_gather_rows, with the
 * same arguments and outputs (cap as for gnf4_hip_route_groups); a_out
 * [T * k, lda] receives the gathered rows of x [T, ldx]. */
int gnf4_hip_route_decode(const float *logits, int64_t ld, int64_t T, int64_t E, int k,
                          int mode, int norm, int64_t *idx, int64_t idx_stride,
                          uint16_t *wts, int64_t wts_stride, const void *x, int64_t ldx,
                          int64_t K, int slots, int cap, int32_t *eids, int32_t *row_off,
                          int32_t *order, int32_t *pos, int32_t *info, void *a_out,
                          int64_t lda, void *stream);

/* out[r, :] = x[order[r] / k, :] (bf16 rows into grouped order;
 * reference arena_moe_patch.py:47 `x[idxs // topk]`). K, ldx, ldo % 8 == 0. */
int gnf4_hip_gather_rows(const void *x, int64_t ldx, const int32_t *order, int64_t N, int k,
                         int64_t K, void *out, int64_t ldo, void *stream);

/* out[t, :] = bf16(sum_j wts[t, j] * y[pos[t * k + j], :]), j ascending in
 * fp32 (the reference's unsort + weight + sum, arena_moe_patch.py:59-65).
 * D, ldy, ldo % 8 == 0. */
int gnf4_hip_route_combine(const void *y, int64_t ldy, const int32_t *pos,
                           const uint16_t *wts, int64_t wts_stride, int64_t T, int k,
                           int64_t D, void *out, int64_t ldo, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GNF4_HIP_H_ */
