/* A C caller linked against libq35mm.so the way the reference's model code
 * links against its matmul (qwen35-c/src/q35_model.c reads the exported
 * table q35_mm_fp8_lut directly, :41-57, after q35_mm_init at :367).
 *
 * Prints the table as hex words before and after q35_mm_init(), then the
 * e4m3 code a nearest-value search over the table picks for each value
 * given on the command line (the search of the reference loader's
 * quantizer: smallest |a - lut[i]| over the 127 finite magnitudes, ties to
 * the even code, sign restored, NaN -> 0x7F). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "q35/q35_mm.h"

static void dump(const char *tag)
{
    printf("%s", tag);
    for (int i = 0; i < 256; i++) {
        uint32_t u;
        memcpy(&u, &q35_mm_fp8_lut[i], 4);
        printf(" %08x", u);
    }
    printf("\n");
}

static unsigned nearest_code(float v)
{
    float a = fabsf(v), best_d = INFINITY;
    unsigned best = 0;
    if (a != a) return 0x7Fu;
    for (unsigned i = 0; i < 128; i++) {
        float lv = q35_mm_fp8_lut[i];
        if (lv != lv) continue;
        float d = fabsf(a - lv);
        if (d < best_d || (d == best_d && (i & 1u) == 0 && (best & 1u))) {
            if (d < best_d) best_d = d;
            best = i;
        }
    }
    return (v < 0.0f ? 0x80u : 0u) | best;
}

int main(int argc, char **argv)
{
    dump("before");
    q35_mm_init();
    dump("after");
    printf("codes");
    for (int i = 1; i < argc; i++) printf(" %u", nearest_code(strtof(argv[i], NULL)));
    printf("\n");
    return 0;
}
