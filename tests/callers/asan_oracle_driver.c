/*
 * asan_oracle_driver.c -- runs the CPU oracle (oracle/fa_oracle.c and its
 * AVX2 / AVX-512 tiers, compiled into this program with AddressSanitizer and
 * UndefinedBehaviorSanitizer) over ragged shapes, block sizes including the
 * 0 clamp and blocks larger than the sequence, causal and non-causal,
 * several heads and thread counts, every available tier, the naive forms and
 * the kernel primitives at odd lengths.  Each v1/v2/v3 output is checked
 * against the f64 naive result (the reference's 1e-3 bar,
 * tests/correctness.rs:109), so the run also fails on wrong numbers.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fa_oracle.h"

static unsigned long long rng = 0x9E3779B97F4A7C15ull;
static float urand(void) {
    rng = rng * 6364136223846793005ull + 1442695040888963407ull;
    return (float)((rng >> 40) & 0xFFFFFF) / 8388608.0f - 1.0f;
}

int main(void) {
    int failures = 0, runs = 0;
    const size_t shapes[][3] = {{1, 1, 1}, {1, 5, 3}, {5, 1, 17}, {17, 23, 32}, {97, 131, 17},
                                {64, 64, 64}, {65, 130, 33}, {200, 37, 129}, {3, 300, 8}};
    const size_t blocks[][2] = {{64, 128}, {0, 0}, {7, 13}, {1, 1}, {512, 1024}};
    for (size_t si = 0; si < sizeof(shapes) / sizeof(shapes[0]); ++si) {
        const size_t sq = shapes[si][0], sk = shapes[si][1], d = shapes[si][2], bh = 1 + si % 3;
        float* q = malloc(bh * sq * d * sizeof(float));
        float* k = malloc(bh * sk * d * sizeof(float));
        float* v = malloc(bh * sk * d * sizeof(float));
        float* o = malloc(bh * sq * d * sizeof(float));
        double* ref = malloc(sq * d * sizeof(double));
        for (size_t i = 0; i < bh * sq * d; ++i) q[i] = urand();
        for (size_t i = 0; i < bh * sk * d; ++i) k[i] = urand(), v[i] = urand();
        for (int causal = 0; causal <= 1; ++causal) {
            for (int tier = ORACLE_TIER_SCALAR; tier <= ORACLE_TIER_AVX512; ++tier) {
                if (!oracle_tier_available(tier)) continue;
                for (int variant = 1; variant <= 3; ++variant) {
                    const size_t* b = blocks[(si + (size_t)variant + (size_t)tier) % 5];
                    if (oracle_run(variant, tier, 1 + (int)(si % 4), q, k, v, bh, sq, sk, d, b[0], b[1], causal, o)) {
                        ++failures;
                        continue;
                    }
                    ++runs;
                    for (size_t h = 0; h < bh; ++h) {
                        oracle_naive_f64(q + h * sq * d, k + h * sk * d, v + h * sk * d, sq, sk, d, causal, ref);
                        for (size_t i = 0; i < sq * d; ++i)
                            if (!(fabs((double)o[h * sq * d + i] - ref[i]) < 1e-3)) {
                                fprintf(stderr, "mismatch shape %zu v%d tier %d causal %d\n", si, variant, tier, causal);
                                ++failures;
                                break;
                            }
                    }
                }
            }
            oracle_naive_f32(q, k, v, sq, sk, d, causal, o);
            oracle_naive_f64_rows(q, k, v, sq, sk, d, causal, sq / 2, sq - sq / 2, ref);
        }
        free(q), free(k), free(v), free(o), free(ref);
    }
    /* zero-sized dims leave out untouched */
    float canary[4] = {5, 5, 5, 5}, one[4] = {1, 1, 1, 1};
    oracle_run(2, ORACLE_TIER_AUTO, 0, one, one, one, 1, 0, 4, 1, 64, 128, 0, canary);
    oracle_run(2, ORACLE_TIER_AUTO, 0, one, one, one, 1, 4, 0, 1, 64, 128, 0, canary);
    if (canary[0] != 5 || canary[3] != 5) ++failures;
    if (oracle_run(9, ORACLE_TIER_AUTO, 0, one, one, one, 1, 1, 1, 1, 64, 128, 0, canary) == 0) ++failures;
    /* primitives at odd lengths */
    float x[67], y[67], a[4 * 37], bb[4 * 37], s16[16], acc[4 * 37], p[4 * 9];
    for (int i = 0; i < 67; ++i) x[i] = 40.0f * urand();
    for (int i = 0; i < 4 * 37; ++i) a[i] = urand(), bb[i] = urand(), acc[i] = 0.0f;
    for (int i = 0; i < 36; ++i) p[i] = urand();
    for (int tier = ORACLE_TIER_SCALAR; tier <= ORACLE_TIER_AVX512; ++tier) {
        if (!oracle_tier_available(tier)) continue;
        for (size_t n = 0; n <= 67; ++n) {
            if (tier != ORACLE_TIER_SCALAR) oracle_exp_simd(tier, x, y, n);
            if (n) (void)oracle_k_max_reduce(tier, x, n);
            memcpy(y, x, sizeof(x));
            if (n) (void)oracle_k_sub_exp_sum(tier, y, n, 40.0f);
            if (n <= 37) (void)oracle_k_dot(tier, a, bb, n);
        }
        oracle_k_dot4x4(tier, a, bb, 37, s16);
        oracle_k_pv4(tier, acc, bb, p, 4, 37);
    }
    printf("runs=%d failures=%d\n", runs, failures);
    if (!failures) printf("asan-oracle ok\n");
    return failures ? 1 : 0;
}
