/*
 * q35_oracle.h -- CPU restatement of the qwen35-c FP8-E4M3 128x128
 * block-scaled dequant + matmul (reference: qwen35-c/src/q35_mm.c).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle the HIP
 * implementation in qwen38-in-c_amd/ is compared with.  Only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it; the
 * product path never links, loads or falls back to it.
 *
 * Every function states the reference lines it restates.  The numerics are
 * the reference's, bit for bit: e4m3 -> fp32 from the OCP OFP8 table, one
 * fp32 multiply by the widened bf16 block scale, eight fmaf accumulation
 * lanes (lane j takes columns j mod 8 in increasing order) and a final
 * sequential lane sum j = 0..7.
 */
#ifndef Q35_ORACLE_H
#define Q35_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar decoders (Q/src/q35_mm.c:22-37, :46-52) ---- */
float orc_e4m3_to_f32(uint8_t v);
float orc_bf16_to_f32(uint16_t v);
void orc_fill_lut(float lut[256]);

/* ---- reference quantizer (Q/src/q35_model.c:31-37, :41-57, :325-344) ---- */
uint16_t orc_f32_to_bf16(float f);
uint8_t orc_f32_to_e4m3(float v);
/* Per 128x128 block: scale = bf16(amax/448); codes = e4m3(w / scale),
 * all-zero block -> scale 0 and zero codes.  w is fp32 [rows][cols]. */
void orc_quantize_fp8(const float *w, uint32_t rows, uint32_t cols,
                      uint8_t *codes, uint16_t *scale_bf16);

/* ---- dequant: out[r][c] = lut[W[r][c]] * s[r/128][c/128] (Q/src/q35_mm.c:99,120) */
void orc_dequant(const uint8_t *W, const uint16_t *scale_bf16,
                 uint32_t rows, uint32_t cols, float *out);
void orc_dequant_f32scale(const uint8_t *W, const float *scale,
                          uint32_t rows, uint32_t cols, float *out);

/* ---- matmul entry points (Q/src/q35_mm.c:88-198) ---- */
void orc_mm_fp8(const uint8_t *W, const uint16_t *scale_bf16,
                uint32_t rows, uint32_t cols, const float *x, float *y);
/* Y is token-major [n][rows] (Q/src/q35_mm.c:168). */
void orc_mm_fp8_batch(const uint8_t *W, const uint16_t *scale_bf16,
                      uint32_t rows, uint32_t cols, uint32_t n,
                      const float *X, float *Y);
void orc_mm_fp8_multi4(const uint8_t *const W[4], const uint16_t *const sc[4],
                       const uint32_t rows[4], uint32_t cols,
                       const float *x, float *const y[4]);
/* Same arithmetic as orc_mm_fp8_batch, but only for the listed weight rows:
 * Y[t][i] = row_idx[i] . X[t], Y is [n][nidx].  Used to check large GEMMs on
 * a sample of output columns. */
void orc_mm_fp8_rows(const uint8_t *W, const uint16_t *scale_bf16,
                     uint32_t rows, uint32_t cols, uint32_t n,
                     const float *X, const uint32_t *row_idx, uint32_t nidx,
                     float *Y);
/* fp32-scale variant of the batch matmul (same lane structure). */
void orc_mm_fp8_batch_f32scale(const uint8_t *W, const float *scale,
                               uint32_t rows, uint32_t cols, uint32_t n,
                               const float *X, float *Y);
/* Exact-math check: the same dequantized weights, dot product in double. */
void orc_mm_fp8_f64(const uint8_t *W, const uint16_t *scale_bf16,
                    uint32_t rows, uint32_t cols, uint32_t n,
                    const float *X, double *Y);

/* ---- BF16 matvec (Q/src/q35_mm.c:211-246): 8 fmaf lanes, no scale ---- */
void orc_mm_bf16(const uint16_t *W, uint32_t rows, uint32_t cols,
                 const float *x, float *y);

/* ---- device-resident neighbours of the MLP (Q/src/q35_kern.c) ----
 * Same operation sequence as the reference's kernels, with FP contraction
 * off (Q/src/q35_kern.c:8): every multiply, add and divide rounds on its own.
 * rmsnorm: sum of squares in eight lanes (element i into lane i mod 8, in
 * increasing i), lanes folded 0..7; mean = s/(float)n;
 * inv = 1/sqrtf(mean + eps); y[i] = (x[i]*inv) * (1 + w[i])
 * (Q/src/q35_kern.c:26-48, :77-86).  rows independent rows of n.
 * silu: x * (1 / (1 + expf(-x)))                      (:70-73, :112-116)
 * swiglu: (g * (1 / (1 + expf(-g)))) * u               (:137-145)
 * add: x[i] = x[i] + y[i], the residual update        (Q/src/q35_model.c:939) */
void orc_rmsnorm(const float *x, const float *w, float *y, uint32_t rows,
                 uint32_t n, float eps);
void orc_silu(const float *x, float *y, size_t n);
void orc_swiglu(const float *gate, const float *up, float *y, size_t n);
void orc_add_inplace(float *x, const float *y, size_t n);
/* libm expf of each element (the function the reference's sigmoid calls). */
void orc_expf(const float *x, float *y, size_t n);

/* ---- hashes used by the reference tests (Q/tests/test_mm.c:19-23,
 *      Q/include/q35/q35_kern.h:77-78) ---- */
uint64_t orc_fnv1a64(const void *p, size_t n);
uint32_t orc_fnv1a32(const void *p, size_t n);
/* FNV-1a-64 variant printed by Q/tests/test_mm.c:19-23 (offset basis
 * 1469598103934665603). */
uint64_t orc_fnv1a64_q35test(const void *p, size_t n);

/* Number of OpenMP threads the oracle runs with (1 without OpenMP). */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
