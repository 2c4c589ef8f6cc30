/* host_token.c -- times a sequence of drop-in q35_mm_* calls on host pointers,
 * as a C caller makes them (the reference model's decode token calls
 * q35_mm_fp8 / q35_mm_fp8_multi4 one after another: qwen35-c/src/q35_model.c:
 * 877-947, qwen35-c/src/q35_deltanet.c:325-329,360, qwen35-c/src/q35_attn.c:
 * 262,273-275).  A benchmark helper: bench.py fills the call list and calls
 * q35_host_calls_time through ctypes once per measurement, so no Python runs
 * between the calls.  Built into lib/libq35host_token.so, linked to
 * libq35mm.so. */
#include <stdint.h>
#include <time.h>

#include "q35/q35_mm.h"

typedef struct q35_host_call {
    uint32_t kind;            /* 0: q35_mm_fp8(W[0]), 1: q35_mm_fp8_multi4(W[0..3]),
                                 2: q35_mm_fp8_batch(W[0]) over rows[1] tokens */
    uint32_t cols;
    const uint8_t *W[4];
    const uint16_t *sc[4];
    uint32_t rows[4];         /* multi4: 0 = segment unused */
    const float *x;
    float *y[4];
} q35_host_call;

static double now_us(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e6 + (double)t.tv_nsec * 1e-3;
}

static void run_calls(const q35_host_call *calls, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        const q35_host_call *c = &calls[i];
        if (c->kind == 0) {
            q35_mm_fp8(c->W[0], c->sc[0], c->rows[0], c->cols, c->x, c->y[0]);
        } else if (c->kind == 2) {
            q35_mm_fp8_batch(c->W[0], c->sc[0], c->rows[0], c->cols, c->rows[1], c->x, c->y[0]);
        } else {
            const uint8_t *W[4] = {c->W[0], c->W[1], c->W[2], c->W[3]};
            const uint16_t *sc[4] = {c->sc[0], c->sc[1], c->sc[2], c->sc[3]};
            uint32_t rows[4] = {c->rows[0], c->rows[1], c->rows[2], c->rows[3]};
            float *y[4] = {c->y[0], c->y[1], c->y[2], c->y[3]};
            q35_mm_fp8_multi4(W, sc, rows, c->cols, c->x, y);
        }
    }
}

/* Runs the list `warmup` times untimed, then `reps` times; returns the mean
 * microseconds of one pass of the list. */
__attribute__((visibility("default"))) double q35_host_calls_time(const q35_host_call *calls, uint32_t n,
                                                                  uint32_t warmup, uint32_t reps) {
    for (uint32_t r = 0; r < warmup; r++) run_calls(calls, n);
    const double t0 = now_us();
    for (uint32_t r = 0; r < reps; r++) run_calls(calls, n);
    return reps ? (now_us() - t0) / reps : 0.0;
}
