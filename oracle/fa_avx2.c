/*
 * fa_avx2.c -- AVX2+FMA tier of the oracle's kernel primitives
 * (restates src/avx2.rs; 8 lanes).  TEST INFRASTRUCTURE ONLY.
 * Only reached after runtime "avx2" and "fma" checks.
 */
#include <immintrin.h>
#include "fa_kernel_ops.h"

#define TIER_ATTR __attribute__((target("avx2,fma")))
#define TIER_SUFFIX _avx2
#define OPS_NAME fa_ops_avx2
#define VEC __m256
#define W 8
#define VLOAD(p) _mm256_loadu_ps(p)
#define VSTORE(p, v) _mm256_storeu_ps((p), (v))
#define VSET1(x) _mm256_set1_ps(x)
#define VZERO() _mm256_setzero_ps()
#define VADD(a, b) _mm256_add_ps((a), (b))
#define VSUB(a, b) _mm256_sub_ps((a), (b))
#define VMUL(a, b) _mm256_mul_ps((a), (b))
#define VFMA(a, b, c) _mm256_fmadd_ps((a), (b), (c))
#define VMAX(a, b) _mm256_max_ps((a), (b))
#define VMIN(a, b) _mm256_min_ps((a), (b))
#define VFLOOR(a) _mm256_floor_ps(a)
#define VPOW2N(fx) \
    _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_add_epi32(_mm256_cvttps_epi32(fx), _mm256_set1_epi32(0x7f)), 23))

/* Horizontal sum / max: fold the two 128-bit halves, then within the half
 * (src/avx2.rs:108-130). */
__attribute__((target("avx2,fma"))) static inline float hsum_avx2(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_extractf128_ps(v, 1), _mm256_castps256_ps128(v));
    __m128 sh = _mm_movehdup_ps(s);
    __m128 t = _mm_add_ps(s, sh);
    __m128 sh2 = _mm_movehl_ps(sh, t);
    return _mm_cvtss_f32(_mm_add_ss(t, sh2));
}
__attribute__((target("avx2,fma"))) static inline float hmax_avx2(__m256 v) {
    __m128 s = _mm_max_ps(_mm256_extractf128_ps(v, 1), _mm256_castps256_ps128(v));
    __m128 sh = _mm_movehdup_ps(s);
    __m128 t = _mm_max_ps(s, sh);
    __m128 sh2 = _mm_movehl_ps(sh, t);
    return _mm_cvtss_f32(_mm_max_ss(t, sh2));
}
#define VHSUM(v) hsum_avx2(v)
#define VHMAX(v) hmax_avx2(v)

#include "fa_simd.inc"
