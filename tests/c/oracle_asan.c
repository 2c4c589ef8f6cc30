/* Drives the oracle's batch and row-subset matmuls under AddressSanitizer on
 * a shape whose K spans more than 1024 scale blocks (the longest K any
 * GEMM test uses), with a last 128-row group that is partial.  Checks:
 *   - orc_mm_fp8_rows(idx) equals the idx columns of orc_mm_fp8_batch bit
 *     for bit (the same dot products on a row subset);
 *   - orc_mm_fp8_batch is within 1e-5 normwise of the float64 dot product of
 *     the same dequantized weights (orc_mm_fp8_f64).
 * Prints "ok" and exits 0, or prints what differs and exits 1; an
 * out-of-bounds access aborts through the sanitizer. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "q35_oracle.h"

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint32_t next32(void)
{
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return (uint32_t)(rng >> 16);
}

int main(int argc, char **argv)
{
    const uint32_t kb = argc > 1 ? (uint32_t)atoi(argv[1]) : 1025u;
    const uint32_t rows = 130, cols = kb * 128u - 5u, n = 2;
    const uint32_t nb = (rows + 127u) / 128u;
    uint8_t *W = malloc((size_t)rows * cols);
    uint16_t *sc = malloc((size_t)nb * kb * 2u);
    float *X = malloc((size_t)n * cols * 4u), *Y = malloc((size_t)n * rows * 4u);
    double *Yd = malloc((size_t)n * rows * 8u);
    uint32_t idx[5] = {0u, 7u, 127u, 128u, 129u};
    float Yr[2 * 5];
    if (!W || !sc || !X || !Y || !Yd) return 2;
    for (size_t i = 0; i < (size_t)rows * cols; i++) {
        uint8_t c = (uint8_t)next32();
        W[i] = (c & 0x7Fu) == 0x7Fu ? (uint8_t)(c - 1u) : c;   /* no NaN codes */
    }
    for (size_t i = 0; i < (size_t)nb * kb; i++) sc[i] = (uint16_t)(0x3A00u + (next32() & 0x3FFu));
    for (size_t i = 0; i < (size_t)n * cols; i++) X[i] = ((float)(next32() & 0xFFFFu) - 32768.0f) / 32768.0f;
    orc_mm_fp8_batch(W, sc, rows, cols, n, X, Y);
    orc_mm_fp8_rows(W, sc, rows, cols, n, X, idx, 5u, Yr);
    orc_mm_fp8_f64(W, sc, rows, cols, n, X, Yd);
    for (uint32_t t = 0; t < n; t++)
        for (uint32_t i = 0; i < 5; i++)
            if (memcmp(&Yr[t * 5u + i], &Y[(size_t)t * rows + idx[i]], 4) != 0) {
                printf("rows differs from batch at token %u row %u\n", t, idx[i]);
                return 1;
            }
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < (size_t)n * rows; i++) {
        num = fmax(num, fabs((double)Y[i] - Yd[i]));
        den = fmax(den, fabs(Yd[i]));
    }
    if (!(num <= 1e-5 * den)) {
        printf("batch vs f64: normwise %.3g\n", num / den);
        return 1;
    }
    printf("ok kb=%u normwise=%.3g\n", kb, num / den);
    free(W); free(sc); free(X); free(Y); free(Yd);
    return 0;
}
