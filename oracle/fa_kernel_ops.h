/*
 * fa_kernel_ops.h -- the numeric primitives the tiling loops run over.
 *
 * TEST INFRASTRUCTURE ONLY (see fa_oracle.h).  One table per tier restates
 * the reference's `Kernel` trait (src/kernel.rs:28-98): the tiling loops in
 * fa_oracle.c are written once and call through this table, as run_vN<K>
 * is monomorphised over K in the reference.
 */
#ifndef FA_KERNEL_OPS_H
#define FA_KERNEL_OPS_H

#include <stddef.h>

typedef struct fa_kernel_ops {
    /* dot(a, b)                                   src/kernel.rs:30 */
    float (*dot)(const float* a, const float* b, size_t n);
    /* [dot(a0,b) .. dot(a3,b)], shared b loads    src/kernel.rs:38 */
    void (*dot4)(const float* a0, const float* a1, const float* a2, const float* a3,
                 const float* b, size_t n, float out[4]);
    /* out[r][c] = dot(q[r], k[c])                 src/kernel.rs:49 */
    void (*dot4x4)(const float* const q[4], const float* const k[4], size_t n, float out[4][4]);
    /* x = exp(x - m) in place, returns sum        src/kernel.rs:55 */
    float (*sub_exp_sum)(float* x, size_t n, float m);
    /* dst += src * s                              src/kernel.rs:58 */
    void (*axpy)(float* dst, const float* src, size_t n, float s);
    /* acc[r][:] += sum_j p[r][j] * v[j][:]        src/kernel.rs:76 */
    void (*pv4)(float* const acc[4], const float* v, const float* const p[4], size_t bc, size_t d);
    /* dst *= s                                    src/kernel.rs:79 */
    void (*scale)(float* dst, size_t n, float s);
    /* max over x, -inf for n == 0                 src/kernel.rs:82 */
    float (*max_reduce)(const float* x, size_t n);
    /* 4 interleaved max reductions                src/kernel.rs:93 */
    void (*max_reduce4)(const float* const x[4], size_t n, float out[4]);
    /* 4 interleaved sub_exp_sum                   src/kernel.rs:97 */
    void (*sub_exp_sum4)(float* const x[4], size_t n, const float m[4], float out[4]);
    /* the tier's vectorised exp, lane-wise (test hook) */
    void (*exp_vec)(const float* x, float* y, size_t n);
} fa_kernel_ops;

extern const fa_kernel_ops fa_ops_scalar;
extern const fa_kernel_ops fa_ops_avx2;
extern const fa_kernel_ops fa_ops_avx512;

#endif
