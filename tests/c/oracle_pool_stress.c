/* Stress test of the oracle's persistent worker pool: many small row-parallel
 * GEMVs whose thread counts alternate between large and small, so that most
 * workers sit each small job out while the next call is already being
 * published. Every result must equal the one-thread result bit for bit.
 * Built and run by tests/test_oracle_pool.py, plain and under
 * ThreadSanitizer. Exit status 0: every call agreed. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/wpc_oracle.h"

static uint64_t rng = 0x9E3779B97F4A7C15ull;
static uint32_t next_u32(void)
{
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return (uint32_t)(rng >> 16);
}

int main(int argc, char** argv)
{
    const int iters = argc > 1 ? atoi(argv[1]) : 2000;
    const size_t rows = 256, cols = 512, nb = cols / 128;
    uint8_t* blocks = malloc(rows * nb * 68);
    float* x = malloc(cols * sizeof(float));
    float* ref = malloc(rows * sizeof(float));
    float* y = malloc(rows * sizeof(float));
    for (size_t b = 0; b < rows * nb; b++) {
        uint8_t* p = blocks + b * 68;
        const uint16_t zp = 0xA7AE, scale = 0x1C19; /* f16 -0.0294, 0.00392 */
        memcpy(p, &zp, 2);
        memcpy(p + 2, &scale, 2);
        for (int j = 0; j < 64; j++) p[4 + j] = (uint8_t)next_u32();
    }
    for (size_t i = 0; i < cols; i++) x[i] = (float)((int)(next_u32() % 2001) - 1000) / 500.0f;
    or_linear_v4_matvec(blocks, rows, cols, x, NULL, ref, 1, 1);
    static const int threads[] = {16, 3, 8, 2, 5, 1, 12, 4, 16, 2};
    const int nt = (int)(sizeof threads / sizeof threads[0]);
    for (int it = 0; it < iters; it++) {
        memset(y, 0xFF, rows * sizeof(float));
        or_linear_v4_matvec(blocks, rows, cols, x, NULL, y, 1, threads[it % nt]);
        if (memcmp(y, ref, rows * sizeof(float)) != 0) {
            fprintf(stderr, "call %d on %d threads differs from the one-thread result\n", it,
                    threads[it % nt]);
            return 1;
        }
    }
    printf("%d calls agree\n", iters);
    free(blocks); free(x); free(ref); free(y);
    return 0;
}
