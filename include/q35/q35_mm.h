/*
 * q35_mm.h -- drop-in C ABI of the qwen35-c FP8 / BF16 matmul, implemented
 * on MI355X (gfx950) by libq35mm.so.
 *
 * Every declaration below keeps the exact C signature and link name of the
 * reference header qwen35-c/include/q35/q35_mm.h, so the model forward
 * (qwen35-c/src/q35_model.c, q35_deltanet.c, q35_attn.c) links against this
 * library unchanged.  Each declaration cites the reference line it replaces.
 *
 * Semantics kept from the reference:
 *   - W is row-major [rows][cols] e4m3fn bytes; scale_bf16 is row-major
 *     [ceil(rows/128)][ceil(cols/128)] bf16 bits, one per 128x128 block.
 *   - x is fp32 [cols]; y is fp32 [rows].  The batch output is token-major:
 *     Y[t][r] for t < n (qwen35-c/src/q35_mm.c:168).
 *   - Calls are synchronous: y is complete when the call returns.
 *   - rows == 0 is a no-op; cols == 0 writes zeros.
 *
 * What differs, by design:
 *   - W and scale_bf16 are uploaded to HBM once, on first use, and stay
 *     resident; later calls with the same pointers reuse the resident copy.
 *     The library detects a changed buffer behind a reused pointer from a
 *     sampled fingerprint; q35mm_release() (q35mm/q35mm.h) drops a copy.
 *   - A HIP failure prints a message on stderr and aborts the process; no
 *     entry point ever returns a partially written y.
 *   - Summation order: fp32 accumulation on the matrix cores instead of the
 *     reference's eight fmaf lanes, so outputs agree to fp32 rounding
 *     (normwise relative difference below 1e-5), not bit for bit.  For
 *     n >= Q35MM_GEMM_MIN_M tokens (default 64) the batch call uses the bf16
 *     prefill GEMM (activations rounded to bf16, fp32 accumulation).
 */
#ifndef Q35_MM_H
#define Q35_MM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* e4m3fn code -> fp32 table, 256 entries; filled at library load and by
 * q35_mm_init.  Replaces qwen35-c/include/q35/q35_mm.h:16. */
extern float q35_mm_fp8_lut[256];

/* Fills q35_mm_fp8_lut (idempotent, thread-safe).  Does not touch the GPU.
 * Replaces qwen35-c/include/q35/q35_mm.h:17. */
void q35_mm_init(void);

/* OCP e4m3fn decode; 0x7F / 0xFF are NaN.  Replaces q35_mm.h:19. */
float q35_mm_e4m3_to_f32(uint8_t v);

/* bf16 storage bits -> fp32, exact.  Replaces q35_mm.h:22. */
float q35_mm_bf16_to_f32(uint16_t v);

/* y[r] = sum_c e4m3(W[r][c]) * scale[r/128][c/128] * x[c].
 * Replaces qwen35-c/include/q35/q35_mm.h:24-26. */
void q35_mm_fp8(const uint8_t *W, const uint16_t *scale_bf16,
                uint32_t rows, uint32_t cols,
                const float *x, float *y);

/* Y[t][r] = row_r . X[t] for t < n; X is [n][cols], Y is [n][rows].
 * Replaces qwen35-c/include/q35/q35_mm.h:32-34. */
void q35_mm_fp8_batch(const uint8_t *W, const uint16_t *scale_bf16,
                      uint32_t rows, uint32_t cols, uint32_t n,
                      const float *X, float *Y);

/* Up to four matrices sharing x and cols, rows[s] == 0 skips segment s;
 * computed in one launch.  Replaces qwen35-c/include/q35/q35_mm.h:40-42. */
void q35_mm_fp8_multi4(const uint8_t *W[4], const uint16_t *sc[4],
                       uint32_t rows[4], uint32_t cols,
                       const float *x, float *y[4]);

/* BF16 matvec y[r] = sum_c bf16(W[r][c]) * x[c].
 * Replaces qwen35-c/include/q35/q35_mm.h:44-45. */
void q35_mm_bf16(const uint16_t *W, uint32_t rows, uint32_t cols,
                 const float *x, float *y);

/* Name of the implementation ("hip-gfx950").  Does not touch the GPU.
 * Replaces qwen35-c/include/q35/q35_mm.h:48. */
const char *q35_mm_impl_fp8(void);

#ifdef __cplusplus
}
#endif

#endif
