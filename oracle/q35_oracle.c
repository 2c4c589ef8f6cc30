/*
 * q35_oracle.c -- CPU restatement of the qwen35-c FP8 block-dequant matmul
 * and of its MLP neighbours (RMSNorm, SiLU, SwiGLU, residual add).
 *
 * TEST INFRASTRUCTURE ONLY (see q35_oracle.h).  Compiled without FP
 * contraction so every multiply and every fmaf rounds exactly as the
 * reference's scalar path does (Q/src/q35_mm.c:4, Q/include/q35/q35_mm.h:11-13).
 *
 * Citations are relative to the reference tree; Q = qwen35-c.
 */
#pragma STDC FP_CONTRACT OFF

#include "q35_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#if defined(_OPENMP)
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Decoders                                                            */
/* ------------------------------------------------------------------ */

static float f32_from_bits(uint32_t u)
{
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static uint32_t bits_from_f32(float f)
{
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* OCP OFP8 E4M3 ("e4m3fn"): 1 sign, 4 exponent bits with bias 7, 3 mantissa
 * bits; no infinities; S.1111.111 is NaN.  Exponent field 0 encodes the
 * subnormals m * 2^-9.  Follows Q/src/q35_mm.c:22-37, including the NaN
 * sign (the reference negates NAN for the 0xFF code). */
float orc_e4m3_to_f32(uint8_t v)
{
    uint32_t sign = (uint32_t)(v >> 7) << 31;
    uint32_t e = (v >> 3) & 0xFu;
    uint32_t m = v & 0x7u;
    if (e == 0) {
        /* m * 2^-9 is exact in fp32; 2^-9 is a power of two. */
        float f = (float)m * 0x1.0p-9f;
        return sign ? -f : f;
    }
    if (e == 15 && m == 7)
        return f32_from_bits(sign | 0x7FC00000u);
    /* value = (1 + m/8) * 2^(e-7): rebias 7 -> 127 and widen the mantissa. */
    return f32_from_bits(sign | ((e + 120u) << 23) | (m << 20));
}

/* bf16 storage bits are the top half of an fp32 (Q/src/q35_mm.c:46-52). */
float orc_bf16_to_f32(uint16_t v)
{
    return f32_from_bits((uint32_t)v << 16);
}

void orc_fill_lut(float lut[256])
{
    for (int i = 0; i < 256; i++) lut[i] = orc_e4m3_to_f32((uint8_t)i);
}

/* ------------------------------------------------------------------ */
/* Quantizer                                                           */
/* ------------------------------------------------------------------ */

/* Round-to-nearest-even fp32 -> bf16 by adding 0x7FFF plus the lsb of the
 * kept half, as Q/src/q35_model.c:31-37 does (no NaN special case). */
uint16_t orc_f32_to_bf16(float f)
{
    uint32_t u = bits_from_f32(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float g_lut[256];

/* The decode table is filled once when the library is loaded, before any
 * OpenMP region can read it. */
__attribute__((constructor)) static void orc_tables_init(void)
{
    orc_fill_lut(g_lut);
}

/* Nearest e4m3 code by exhaustive search over the 127 finite non-negative
 * magnitudes (codes 0x00..0x7E), keeping the first strictly-closer code and
 * switching to an even code on an exact tie; the sign is taken from v < 0.
 * This is the search of Q/src/q35_model.c:41-57, and it inherits that
 * search's edge behaviour: NaN -> 0x7F, magnitudes above 448 saturate to
 * 0x7E, and -0.0f maps to 0x00. */
uint8_t orc_f32_to_e4m3(float v)
{
    const float *mags = g_lut;   /* codes 0x00..0x7F are the non-negative half */
    if (v != v) return 0x7Fu;
    float a = fabsf(v);
    float best_d = 1e30f;
    int best = 0;
    for (int i = 0; i < 127; i++) {          /* 127 is the NaN code */
        float d = fabsf(a - mags[i]);
        int closer = d < best_d;
        int even_tie = (d == best_d) && !(i & 1) && (best & 1);
        if (closer || even_tie) {
            best_d = d;
            best = i;
        }
    }
    return (uint8_t)((v < 0.0f ? 0x80u : 0x00u) | (uint32_t)best);
}

/* Block quantizer of Q/src/q35_model.c:325-344, applied to fp32 weights:
 * amax over the (possibly partial) 128x128 block, scale = amax / 448 in
 * fp32, rounded to bf16; blocks whose bf16 scale is zero keep zero codes. */
void orc_quantize_fp8(const float *w, uint32_t rows, uint32_t cols,
                      uint8_t *codes, uint16_t *scale_bf16)
{
    uint32_t nb = (rows + 127u) / 128u, kb = (cols + 127u) / 128u;
    memset(codes, 0, (size_t)rows * cols);
    #pragma omp parallel for schedule(static)
    for (int64_t blk = 0; blk < (int64_t)nb * kb; blk++) {
        uint32_t bi = (uint32_t)(blk / kb), bj = (uint32_t)(blk % kb);
        uint32_t r0 = bi * 128u, c0 = bj * 128u;
        uint32_t r1 = r0 + 128u < rows ? r0 + 128u : rows;
        uint32_t c1 = c0 + 128u < cols ? c0 + 128u : cols;
        float amax = 0.0f;
        for (uint32_t r = r0; r < r1; r++)
            for (uint32_t c = c0; c < c1; c++) {
                float a = fabsf(w[(size_t)r * cols + c]);
                if (a > amax) amax = a;
            }
        uint16_t sb = orc_f32_to_bf16(amax / 448.0f);
        float s = orc_bf16_to_f32(sb);
        scale_bf16[(size_t)bi * kb + bj] = sb;
        if (s == 0.0f) continue;
        for (uint32_t r = r0; r < r1; r++)
            for (uint32_t c = c0; c < c1; c++)
                codes[(size_t)r * cols + c] =
                    orc_f32_to_e4m3(w[(size_t)r * cols + c] / s);
    }
}

/* ------------------------------------------------------------------ */
/* Dequant                                                             */
/* ------------------------------------------------------------------ */

static const float *lut(void)
{
    return g_lut;
}

void orc_dequant(const uint8_t *W, const uint16_t *scale_bf16,
                 uint32_t rows, uint32_t cols, float *out)
{
    const float *L = lut();
    uint32_t kb = (cols + 127u) / 128u;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++)
        for (uint32_t c = 0; c < cols; c++) {
            float s = orc_bf16_to_f32(scale_bf16[(size_t)(r / 128) * kb + c / 128]);
            out[(size_t)r * cols + c] = L[W[(size_t)r * cols + c]] * s;
        }
}

void orc_dequant_f32scale(const uint8_t *W, const float *scale,
                          uint32_t rows, uint32_t cols, float *out)
{
    const float *L = lut();
    uint32_t kb = (cols + 127u) / 128u;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++)
        for (uint32_t c = 0; c < cols; c++) {
            float s = scale[(size_t)(r / 128) * kb + c / 128];
            out[(size_t)r * cols + c] = L[W[(size_t)r * cols + c]] * s;
        }
}

/* ------------------------------------------------------------------ */
/* Matmul                                                              */
/* ------------------------------------------------------------------ */

/* One output of the block-dequant dot product (Q/src/q35_mm.c:88-142, the
 * scalar form, which the reference's AVX2 form reproduces bit for bit):
 * for each 128-column block the widened scale s is fetched once; every
 * weight is lut[b] * s (one rounded fp32 multiply) and enters
 * acc[c mod 8] through fmaf; the eight lanes are then added in order. */
static float dot_row(const uint8_t *wr, const float *srow, uint32_t cols,
                     const float *x)
{
    const float *L = lut();
    float acc[8] = { 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f };
    for (uint32_t c0 = 0; c0 < cols; c0 += 128u) {
        uint32_t c1 = c0 + 128u < cols ? c0 + 128u : cols;
        float s = srow[c0 / 128u];
        for (uint32_t c = c0; c < c1; c++) {
            float wv = L[wr[c]] * s;
            acc[c & 7u] = fmaf(wv, x[c], acc[c & 7u]);
        }
    }
    float sum = 0.f;
    for (int j = 0; j < 8; j++) sum += acc[j];
    return sum;
}

/* A thread's buffer for one widened scale row (kb floats); aborts when the
 * allocation fails, so no caller ever runs on a short buffer. */
static float *scale_row_alloc(uint32_t kb)
{
    float *p = (float *)malloc((size_t)(kb ? kb : 1u) * sizeof(float));
    if (!p) {
        fprintf(stderr, "oracle: out of memory for a scale row of %u blocks\n", kb);
        abort();
    }
    return p;
}

/* Widened scale row for weight row r: s[r/128][*] as fp32. */
static void scale_row_bf16(const uint16_t *sc, uint32_t r, uint32_t kb, float *srow)
{
    for (uint32_t j = 0; j < kb; j++)
        srow[j] = orc_bf16_to_f32(sc[(size_t)(r / 128u) * kb + j]);
}

void orc_mm_fp8_batch(const uint8_t *W, const uint16_t *scale_bf16,
                      uint32_t rows, uint32_t cols, uint32_t n,
                      const float *X, float *Y)
{
    uint32_t kb = (cols + 127u) / 128u;
    #pragma omp parallel
    {
        float *srow = scale_row_alloc(kb);
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < (int64_t)rows; r++) {
            scale_row_bf16(scale_bf16, (uint32_t)r, kb, srow);
            for (uint32_t t = 0; t < n; t++)
                Y[(size_t)t * rows + (size_t)r] =
                    dot_row(W + (size_t)r * cols, srow, cols, X + (size_t)t * cols);
        }
        free(srow);
    }
}

void orc_mm_fp8(const uint8_t *W, const uint16_t *scale_bf16,
                uint32_t rows, uint32_t cols, const float *x, float *y)
{
    orc_mm_fp8_batch(W, scale_bf16, rows, cols, 1u, x, y);
}

/* Up to four matrices sharing x and cols (Q/src/q35_mm.c:176-198); each
 * segment's rows are the same dot products as a single call. */
void orc_mm_fp8_multi4(const uint8_t *const W[4], const uint16_t *const sc[4],
                       const uint32_t rows[4], uint32_t cols,
                       const float *x, float *const y[4])
{
    for (int s = 0; s < 4; s++)
        if (rows[s]) orc_mm_fp8(W[s], sc[s], rows[s], cols, x, y[s]);
}

void orc_mm_fp8_rows(const uint8_t *W, const uint16_t *scale_bf16,
                     uint32_t rows, uint32_t cols, uint32_t n,
                     const float *X, const uint32_t *row_idx, uint32_t nidx,
                     float *Y)
{
    (void)rows;
    uint32_t kb = (cols + 127u) / 128u;
    #pragma omp parallel
    {
        float *srow = scale_row_alloc(kb);
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < (int64_t)nidx; i++) {
            uint32_t r = row_idx[i];
            scale_row_bf16(scale_bf16, r, kb, srow);
            for (uint32_t t = 0; t < n; t++)
                Y[(size_t)t * nidx + (size_t)i] =
                    dot_row(W + (size_t)r * cols, srow, cols, X + (size_t)t * cols);
        }
        free(srow);
    }
}

void orc_mm_fp8_batch_f32scale(const uint8_t *W, const float *scale,
                               uint32_t rows, uint32_t cols, uint32_t n,
                               const float *X, float *Y)
{
    uint32_t kb = (cols + 127u) / 128u;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        const float *srow = scale + (size_t)(r / 128) * kb;
        for (uint32_t t = 0; t < n; t++)
            Y[(size_t)t * rows + (size_t)r] =
                dot_row(W + (size_t)r * cols, srow, cols, X + (size_t)t * cols);
    }
}

void orc_mm_fp8_f64(const uint8_t *W, const uint16_t *scale_bf16,
                    uint32_t rows, uint32_t cols, uint32_t n,
                    const float *X, double *Y)
{
    const float *L = lut();
    uint32_t kb = (cols + 127u) / 128u;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++)
        for (uint32_t t = 0; t < n; t++) {
            double acc = 0.0;
            const float *x = X + (size_t)t * cols;
            for (uint32_t c = 0; c < cols; c++) {
                float s = orc_bf16_to_f32(scale_bf16[(size_t)(r / 128) * kb + c / 128]);
                acc += (double)(L[W[(size_t)r * cols + c]] * s) * (double)x[c];
            }
            Y[(size_t)t * rows + (size_t)r] = acc;
        }
}

/* BF16 matvec with the same eight-lane fmaf structure and no scales
 * (Q/src/q35_mm.c:211-246). */
void orc_mm_bf16(const uint16_t *W, uint32_t rows, uint32_t cols,
                 const float *x, float *y)
{
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        const uint16_t *wr = W + (size_t)r * cols;
        float acc[8] = { 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f };
        for (uint32_t c = 0; c < cols; c++)
            acc[c & 7u] = fmaf(orc_bf16_to_f32(wr[c]), x[c], acc[c & 7u]);
        float sum = 0.f;
        for (int j = 0; j < 8; j++) sum += acc[j];
        y[r] = sum;
    }
}

/* ------------------------------------------------------------------ */
/* MLP neighbours (Q/src/q35_kern.c)                                    */
/* ------------------------------------------------------------------ */

/* Q/src/q35_kern.c:26-48 (sumsq_fixed) and :77-86 (q35_kern_rmsnorm_scalar).
 * The AVX2 variants (:29-38, :88-108) run the same operations lane for lane;
 * the reference's test checks the two paths hash-equal. */
void orc_rmsnorm(const float *x, const float *w, float *y, uint32_t rows,
                 uint32_t n, float eps)
{
    #pragma omp parallel for schedule(static) if (rows > 1)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        const float *xr = x + (size_t)r * n;
        float *yr = y + (size_t)r * n;
        float lane[8] = { 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f };
        for (uint32_t i = 0; i < n; i++) {
            const float sq = xr[i] * xr[i];
            lane[i % 8u] = lane[i % 8u] + sq;
        }
        float s = lane[0];
        for (int j = 1; j < 8; j++) s = s + lane[j];
        const float mean = s / (float)n;
        const float inv = 1.0f / sqrtf(mean + eps);
        for (uint32_t i = 0; i < n; i++) {
            const float t = xr[i] * inv;
            yr[i] = t * (1.0f + w[i]);
        }
    }
}

/* Q/src/q35_kern.c:70-73 (sigmoidf_). */
static float sigmoid_ref(float v)
{
    const float e = expf(-v);
    return 1.0f / (1.0f + e);
}

/* Q/src/q35_kern.c:112-116 (q35_kern_silu_scalar). */
void orc_silu(const float *x, float *y, size_t n)
{
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; i++) y[i] = x[i] * sigmoid_ref(x[i]);
}

/* Q/src/q35_kern.c:137-145 (the AVX2 variant :147-166 computes the same
 * t = g*sigmoid(g) per element and one multiply by up). */
void orc_swiglu(const float *gate, const float *up, float *y, size_t n)
{
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; i++) {
        const float t = gate[i] * sigmoid_ref(gate[i]);
        y[i] = t * up[i];
    }
}

/* Q/src/q35_model.c:939 and :977 (x[j] += y[j]). */
void orc_add_inplace(float *x, const float *y, size_t n)
{
    for (size_t i = 0; i < n; i++) x[i] = x[i] + y[i];
}

void orc_expf(const float *x, float *y, size_t n)
{
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; i++) y[i] = expf(x[i]);
}

/* ------------------------------------------------------------------ */
/* Hashes                                                              */
/* ------------------------------------------------------------------ */

uint64_t orc_fnv1a64(const void *p, size_t n)
{
    const unsigned char *b = (const unsigned char *)p;
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; i++) {
        h ^= b[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

/* The hash Q/tests/test_mm.c:19-23 prints: FNV-1a-64 with the offset basis
 * written as the decimal 1469598103934665603, which is the standard basis
 * 14695981039346656037 with its last digit dropped.  Kept so the hashes the
 * reference test prints can be compared directly. */
uint64_t orc_fnv1a64_q35test(const void *p, size_t n)
{
    const unsigned char *b = (const unsigned char *)p;
    uint64_t h = 1469598103934665603ull;
    for (size_t i = 0; i < n; i++) {
        h ^= b[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

uint32_t orc_fnv1a32(const void *p, size_t n)
{
    const unsigned char *b = (const unsigned char *)p;
    uint32_t h = 0x811c9dc5u;
    for (size_t i = 0; i < n; i++) {
        h ^= b[i];
        h *= 0x01000193u;
    }
    return h;
}

int orc_num_threads(void)
{
#if defined(_OPENMP)
    return omp_get_max_threads();
#else
    return 1;
#endif
}
