/*
 * fa_avx512.c -- AVX-512F tier of the oracle's kernel primitives
 * (restates src/avx512.rs; 16 lanes).  TEST INFRASTRUCTURE ONLY.
 * Only reached after a runtime __builtin_cpu_supports("avx512f") check.
 */
#include <immintrin.h>
#include "fa_kernel_ops.h"

#define TIER_ATTR __attribute__((target("avx512f")))
#define TIER_SUFFIX _avx512
#define OPS_NAME fa_ops_avx512
#define VEC __m512
#define W 16
#define VLOAD(p) _mm512_loadu_ps(p)
#define VSTORE(p, v) _mm512_storeu_ps((p), (v))
#define VSET1(x) _mm512_set1_ps(x)
#define VZERO() _mm512_setzero_ps()
#define VADD(a, b) _mm512_add_ps((a), (b))
#define VSUB(a, b) _mm512_sub_ps((a), (b))
#define VMUL(a, b) _mm512_mul_ps((a), (b))
#define VFMA(a, b, c) _mm512_fmadd_ps((a), (b), (c))
#define VMAX(a, b) _mm512_max_ps((a), (b))
#define VMIN(a, b) _mm512_min_ps((a), (b))
#define VFLOOR(a) _mm512_roundscale_ps((a), _MM_FROUND_TO_NEG_INF | _MM_FROUND_NO_EXC)
#define VPOW2N(fx) \
    _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_add_epi32(_mm512_cvttps_epi32(fx), _mm512_set1_epi32(0x7f)), 23))
#define VHSUM(v) _mm512_reduce_add_ps(v)
#define VHMAX(v) _mm512_reduce_max_ps(v)

#include "fa_simd.inc"
