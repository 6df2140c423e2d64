/* gnf4_oracle.c -- CPU oracle for the grouped 4-bit expert GEMM.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the GPU kernels are
 * compared against and the CPU baseline that bench.py times beside them. No
 * product code path links or calls it.
 *
 * It restates, in plain C, the locked summation order of the reference's CPU
 * tier (reference: gnf4_native/cpu_kernels.c:15-34 for the forward tree,
 * :1111-1131 for the dgrad chain; numpy mirror kernel/cpu_grouped.py:53-144).
 *
 * Forward (one output element: row r of group g, column n):
 *   K is consumed as 16-lane groups lg = 0, 1, 2, ... ascending. Lane group lg
 *   accumulates into accumulator set lg % 4. Per lane i:
 *       w    = LUT[code] * scale          (one fp32 rounding)
 *       prod = w * a                      (fp32 multiply)
 *       acc[lg % 4][i] += prod            (fp32 add; never fused into an FMA)
 *   then comb[i] = (acc0[i] + acc1[i]) + (acc2[i] + acc3[i]) and a sequential
 *   sum over lanes i = 0..15 starting from 0.0f.
 * dgrad (one output element gi[t, k], caller-zeroed):
 *   for n ascending: w = LUT[code(n,k)] * scale;  p = w * g[t, n];  acc += p.
 *
 * Formats (reference kernel/nf4_grouped.py:53-71, kernel/mxfp4_pack_ref.py:21-70):
 *   NF4   byte j holds elements 2j (HIGH nibble) and 2j+1 (LOW nibble);
 *         scale = absmax[n, k / 64] (fp32).
 *   MXFP4 byte j holds elements 2j (LOW nibble) and 2j+1 (HIGH nibble);
 *         scale = 2^(e - 127) for the e8m0 byte e of block k / 32. e = 0 is the
 *         subnormal 2^-127; e = 255 follows ldexp semantics, w = ldexp(v, 128)
 *         (zero stays zero, anything else becomes +-inf), reference
 *         gnf4_native/cpu_kernels.c:394-402 and :1052-1062.
 *
 * Build with -ffp-contract=off: contraction of mul+add into FMA would change
 * the bits of the locked tree.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_EXPORT __attribute__((visibility("default")))

/* NF4 codebook, reference kernel/nf4_grouped.py:53-71. */
static const float kNf4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f,
};

/* e2m1 codebook, index = sign << 3 | magnitude; reference
 * kernel/mxfp4_pack_ref.py:21-22. */
static const float kFp4[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

enum { FMT_NF4 = 0, FMT_MXFP4 = 1 };

ORACLE_EXPORT const float *gnf4o_nf4_lut(void) { return kNf4; }
ORACLE_EXPORT const float *gnf4o_fp4_lut(void) { return kFp4; }

/* 2^(e - 127) as an fp32 value, exact for e in 0..254 (e = 0 is subnormal). */
static float e8m0_to_f32(unsigned e) {
    if (e == 0) return ldexpf(1.0f, -127);
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)e << 23;
    return v.f;
}

/* Decode elements [k0, k1) of one weight row into w[0 .. k1-k0), elementwise
 * identical to the reference decode (one rounding: LUT * scale, or ldexp for
 * e8m0 == 255). k0 and k1 are even. */
static void decode_span(int fmt, const uint8_t *row, const void *scale_row,
                        int64_t k0, int64_t k1, float *w) {
    if (fmt == FMT_NF4) {
        const float *am = (const float *)scale_row;
        for (int64_t j = k0 / 2; j < k1 / 2; j++) {
            float s = am[(2 * j) / 64];
            uint8_t b = row[j];
            w[2 * j - k0] = kNf4[b >> 4] * s;
            w[2 * j + 1 - k0] = kNf4[b & 15] * s;
        }
    } else {
        const uint8_t *sc = (const uint8_t *)scale_row;
        for (int64_t j = k0 / 2; j < k1 / 2; j++) {
            unsigned e = sc[(2 * j) / 32];
            uint8_t b = row[j];
            float v0 = kFp4[b & 15], v1 = kFp4[b >> 4];
            if (e == 255) {
                w[2 * j - k0] = ldexpf(v0, 128);
                w[2 * j + 1 - k0] = ldexpf(v1, 128);
            } else {
                float s = e8m0_to_f32(e);
                w[2 * j - k0] = v0 * s;
                w[2 * j + 1 - k0] = v1 * s;
            }
        }
    }
}

/* The locked forward tree for one (row, column) pair. */
static float locked_dot(const float *a, const float *w, int64_t K) {
    float acc[4][16];
    memset(acc, 0, sizeof(acc));
    for (int64_t lg = 0; lg < K / 16; lg++) {
        float *dst = acc[lg & 3];
        const float *ap = a + lg * 16, *wp = w + lg * 16;
        for (int i = 0; i < 16; i++) {
            float prod = wp[i] * ap[i];
            dst[i] = dst[i] + prod;
        }
    }
    float s = 0.0f;
    for (int i = 0; i < 16; i++) {
        float c = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
        s = s + c;
    }
    return s;
}

static int check_groups(const int64_t *eids, const int32_t *sizes, int G,
                        int64_t E, int64_t *row_off) {
    int64_t r = 0;
    for (int g = 0; g < G; g++) {
        if (sizes[g] < 0 || eids[g] < 0 || eids[g] >= E) return -1;
        row_off[g] = r;
        r += sizes[g];
    }
    row_off[G] = r;
    return 0;
}

#define COL_TILE 32

/* Grouped forward: out[r, n] = locked_dot(a[r, :], decode(W[e(r)][n, :])).
 *   a      [R, K] fp32, rows sorted by group
 *   packed [E, N, K/2] u8; scales [E, N, K/64] fp32 (NF4) or [E, N, K/32] u8
 *   eids [G] int64; sizes [G] int32 (>= 0; empty groups allowed here)
 *   out    [R, N] fp32
 * Returns 0, or -1 on a shape or group violation. */
ORACLE_EXPORT int gnf4o_gemv_grouped(int fmt, const float *a,
                                     const uint8_t *packed,
                                     const void *scales, const int64_t *eids,
                                     const int32_t *sizes, int G, int64_t E,
                                     int64_t N, int64_t K, float *out,
                                     int threads) {
    int64_t blk = fmt == FMT_NF4 ? 64 : 32;
    if ((fmt != FMT_NF4 && fmt != FMT_MXFP4) || K <= 0 || K % blk || N <= 0 ||
        G < 0 || E <= 0)
        return -1;
    int64_t *row_off = (int64_t *)malloc(sizeof(int64_t) * (size_t)(G + 1));
    if (!row_off) return -2;
    if (check_groups(eids, sizes, G, E, row_off)) {
        free(row_off);
        return -1;
    }
    int64_t tiles_n = (N + COL_TILE - 1) / COL_TILE;
    int64_t total = (int64_t)G * tiles_n;
    size_t scale_row_bytes = fmt == FMT_NF4 ? (size_t)(K / 64) * 4 : (size_t)(K / 32);
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    int failed = 0;
#pragma omp parallel
    {
        float *w = (float *)malloc(sizeof(float) * (size_t)K);
        if (!w) {
#pragma omp atomic write
            failed = 1;
        }
#pragma omp for schedule(static)
        for (int64_t u = 0; u < total; u++) {
            if (!w) continue;
            int g = (int)(u / tiles_n);
            int64_t n0 = (u % tiles_n) * COL_TILE;
            int64_t n1 = n0 + COL_TILE < N ? n0 + COL_TILE : N;
            int64_t e = eids[g];
            for (int64_t n = n0; n < n1; n++) {
                const uint8_t *row = packed + (e * N + n) * (K / 2);
                const char *srow = (const char *)scales +
                                   (size_t)(e * N + n) * scale_row_bytes;
                decode_span(fmt, row, srow, 0, K, w);
                for (int64_t r = row_off[g]; r < row_off[g + 1]; r++)
                    out[r * N + n] = locked_dot(a + r * K, w, K);
            }
        }
        free(w);
    }
    free(row_off);
    return failed ? -2 : 0;
}

#define DG_K_TILE 128

/* Grouped dgrad: gi[t, k] += w[n, k] * g[t, n] for n ascending, into a
 * caller-zeroed out [R, K]. Same layouts as the forward; g is [R, N]. */
ORACLE_EXPORT int gnf4o_dgrad_grouped(int fmt, const float *g,
                                      const uint8_t *packed,
                                      const void *scales, const int64_t *eids,
                                      const int32_t *sizes, int G, int64_t E,
                                      int64_t N, int64_t K, float *out,
                                      int threads) {
    int64_t blk = fmt == FMT_NF4 ? 64 : 32;
    if ((fmt != FMT_NF4 && fmt != FMT_MXFP4) || K <= 0 || K % blk || N <= 0 ||
        G < 0 || E <= 0)
        return -1;
    int64_t *row_off = (int64_t *)malloc(sizeof(int64_t) * (size_t)(G + 1));
    if (!row_off) return -2;
    if (check_groups(eids, sizes, G, E, row_off)) {
        free(row_off);
        return -1;
    }
    size_t scale_row_bytes = fmt == FMT_NF4 ? (size_t)(K / 64) * 4 : (size_t)(K / 32);
    int64_t tiles_k = (K + DG_K_TILE - 1) / DG_K_TILE;
    int64_t total = (int64_t)G * tiles_k;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    int failed = 0;
#pragma omp parallel
    {
        float *w = (float *)malloc(sizeof(float) * (size_t)K);
        if (!w) {
#pragma omp atomic write
            failed = 1;
        }
#pragma omp for schedule(static)
        for (int64_t u = 0; u < total; u++) {
            if (!w) continue;
            int gi = (int)(u / tiles_k);
            int64_t k0 = (u % tiles_k) * DG_K_TILE;
            int64_t k1 = k0 + DG_K_TILE < K ? k0 + DG_K_TILE : K;
            int64_t e = eids[gi];
            for (int64_t n = 0; n < N; n++) {
                const uint8_t *row = packed + (e * N + n) * (K / 2);
                const char *srow = (const char *)scales +
                                   (size_t)(e * N + n) * scale_row_bytes;
                decode_span(fmt, row, srow, k0, k1, w);
                for (int64_t t = row_off[gi]; t < row_off[gi + 1]; t++) {
                    float gv = g[t * N + n];
                    float *o = out + t * K;
                    for (int64_t k = k0; k < k1; k++) {
                        float p = w[k - k0] * gv;
                        o[k] = o[k] + p;
                    }
                }
            }
        }
        free(w);
    }
    free(row_off);
    return failed ? -2 : 0;
}

/* ---------------------------------------------------------------- FFN -- */

/* The locked fp32 silu of the fused expert FFN ("gnf4-silu-horner6/1",
 * reference gnf4_native/cpu_kernels.c:776-822, numpy spec
 * kernel/cpu_grouped.py:147-179). The op sequence is the contract:
 *   x > 87 -> x;  x < -87 -> 0;
 *   t = x * -log2(e);  n = floor(t + 0.5);  f = t - n;
 *   p = degree-6 Horner in f (mul then add, never fused);
 *   e = p * 2^n (exponent bits);  silu = x * (1 / (1 + e)). */
static float silu_locked(float x) {
    if (x > 87.0f) return x;
    if (x < -87.0f) return 0.0f;
    float t = x * -1.442695040888963e0f;
    float n = floorf(t + 0.5f);
    float f = t - n;
    float p = 1.535336188319500e-4f;
    p = p * f + 1.339887440266574e-3f;
    p = p * f + 9.618437357674640e-3f;
    p = p * f + 5.550332471162809e-2f;
    p = p * f + 2.402264791363012e-1f;
    p = p * f + 6.931472028550421e-1f;
    p = p * f + 1.0f;
    union { uint32_t u; float f32; } sc;
    sc.u = (uint32_t)((int32_t)n + 127) << 23;
    float e = p * sc.f32;
    return x * (1.0f / (1.0f + e));
}

ORACLE_EXPORT void gnf4o_silu_locked(const float *x, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = silu_locked(x[i]);
}

/* Fused NF4 expert FFN, spec form (reference kernel/cpu_grouped.py:182-194,
 * C entry gnf4_gemv_nf4_ffn_grouped, cpu_kernels.c:948-986):
 *   gu  = gemv(a, W_gu)                [R, 2H]  locked tree
 *   h   = silu_locked(gu[:, :H]) * gu[:, H:]   (fp32 multiply)
 *   out = gemv(h, W_dn)                [R, N_dn] locked tree
 * The fused form and this composition are the same arithmetic, so the two
 * agree exactly. */
ORACLE_EXPORT int gnf4o_ffn_grouped(const float *a, const uint8_t *gu_packed,
                                    const float *gu_absmax, const uint8_t *dn_packed,
                                    const float *dn_absmax, const int64_t *eids,
                                    const int32_t *sizes, int G, int64_t E,
                                    int64_t N_gu, int64_t K, int64_t N_dn,
                                    float *out, int threads) {
    if (N_gu <= 0 || N_gu % 2 || (N_gu / 2) % 64 || K % 64 || N_dn <= 0 || G < 0)
        return -1;
    int64_t H = N_gu / 2, R = 0;
    for (int g = 0; g < G; g++) {
        if (sizes[g] < 0) return -1;
        R += sizes[g];
    }
    float *gu = (float *)malloc(sizeof(float) * (size_t)(R * N_gu + 1));
    float *h = (float *)malloc(sizeof(float) * (size_t)(R * H + 1));
    int rc = (gu && h) ? 0 : -2;
    if (!rc)
        rc = gnf4o_gemv_grouped(FMT_NF4, a, gu_packed, gu_absmax, eids, sizes, G, E,
                                N_gu, K, gu, threads);
    if (!rc) {
        for (int64_t r = 0; r < R; r++)
            for (int64_t j = 0; j < H; j++) {
                float s = silu_locked(gu[r * N_gu + j]);
                h[r * H + j] = s * gu[r * N_gu + H + j];
            }
        rc = gnf4o_gemv_grouped(FMT_NF4, h, dn_packed, dn_absmax, eids, sizes, G, E,
                                N_dn, H, out, threads);
    }
    free(gu);
    free(h);
    return rc;
}

/* -------------------------------------------------------------- routing -- */

/* Top-k + softmax weights per token, restating the reference's
 * gnf4_route_epilogue_bf16 (gnf4_native/cpu_kernels.c:1408-1471): an
 * insertion selection over ascending e where only a strictly larger value
 * moves an entry up (ties keep the earlier index = stable descending order);
 * mode 0: m = max over all logits, z = sum of expf(l - m) in ascending e,
 * w_j = expf(v_j - m) / z, renormalised by their ascending sum when norm;
 * mode 1: the same over the k selected values; weights to bf16 by
 * round-to-nearest-even. Returns -1 on bad arguments. */
static uint16_t to_bf16_rne(float x) {
    union { float f; uint32_t u; } v = { x };
    return (uint16_t)((v.u + 0x7FFFu + ((v.u >> 16) & 1u)) >> 16);
}

ORACLE_EXPORT int gnf4o_route_topk(const float *logits, int64_t T, int64_t E, int64_t k,
                                   int mode, int norm, int64_t *idx, uint16_t *wts) {
    if (k < 1 || k > 64 || k > E || (mode != 0 && mode != 1)) return -1;
    for (int64_t t = 0; t < T; t++) {
        const float *lg = logits + t * E;
        float val[64];
        int64_t id[64];
        int64_t n = 0;
        for (int64_t e = 0; e < E; e++) {
            float x = lg[e];
            int64_t slot;
            if (n < k) {
                slot = n++;
            } else if (x > val[k - 1]) {
                slot = k - 1;
            } else {
                continue;
            }
            while (slot > 0 && val[slot - 1] < x) {
                val[slot] = val[slot - 1];
                id[slot] = id[slot - 1];
                slot--;
            }
            val[slot] = x;
            id[slot] = e;
        }
        float w[64];
        if (mode == 0) {
            float m = lg[0];
            for (int64_t e = 1; e < E; e++)
                if (lg[e] > m) m = lg[e];
            float z = 0.0f;
            for (int64_t e = 0; e < E; e++) z += expf(lg[e] - m);
            for (int64_t j = 0; j < k; j++) w[j] = expf(val[j] - m) / z;
            if (norm) {
                float s = 0.0f;
                for (int64_t j = 0; j < k; j++) s += w[j];
                for (int64_t j = 0; j < k; j++) w[j] /= s;
            }
        } else {
            float z = 0.0f;
            for (int64_t j = 0; j < k; j++) z += expf(val[j] - val[0]);
            for (int64_t j = 0; j < k; j++) w[j] = expf(val[j] - val[0]) / z;
        }
        for (int64_t j = 0; j < k; j++) {
            idx[t * k + j] = id[j];
            wts[t * k + j] = to_bf16_rne(w[j]);
        }
    }
    return 0;
}

/* Grouping of the N = T * k routed rows by expert (the MoE dispatch's
 * stable sort by expert id, reference kernel/arena_moe_patch.py:41-47):
 * counts per expert, groups = experts with rows in ascending id order,
 * row_off = exclusive prefix of the counts, order = rows in (expert, row)
 * order, pos = its inverse. Returns the number of groups, or -1 for an id
 * outside [0, E). */
ORACLE_EXPORT int gnf4o_route_groups(const int64_t *ids, int64_t N, int64_t E, int32_t *eids,
                                     int32_t *row_off, int32_t *order, int32_t *pos) {
    int64_t *cnt = (int64_t *)calloc((size_t)E + 1, sizeof(int64_t));
    if (!cnt) return -2;
    for (int64_t i = 0; i < N; i++) {
        if (ids[i] < 0 || ids[i] >= E) {
            free(cnt);
            return -1;
        }
        cnt[ids[i]]++;
    }
    int g = 0;
    int64_t base = 0;
    int64_t *start = (int64_t *)malloc(sizeof(int64_t) * (size_t)(E + 1));
    if (!start) {
        free(cnt);
        return -2;
    }
    for (int64_t e = 0; e < E; e++) {
        start[e] = base;
        if (cnt[e]) {
            eids[g] = (int32_t)e;
            row_off[g] = (int32_t)base;
            g++;
        }
        base += cnt[e];
    }
    row_off[g] = (int32_t)base;
    for (int64_t i = 0; i < N; i++) {
        int64_t p = start[ids[i]]++;
        order[p] = (int32_t)i;
        pos[i] = (int32_t)p;
    }
    free(start);
    free(cnt);
    return g;
}
