/*
 * fa_oracle.h -- CPU restatement of the reference crate's FlashAttention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker and the timed
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product (libfa_hip.so) never links,
 * loads or calls it, and there is no CPU fallback in the product path.
 *
 * What it restates (all citations into the reference, amaye15/flash-attention-cpu):
 *   - naive_attention                 src/naive.rs:14-75
 *   - run_v1 (FA-1 tiling)            src/v1.rs:162-396
 *   - run_v2 (FA-2 tiling, the oracle) src/v2.rs:160-385
 *   - run_v3 (pipelined v2)           src/v3.rs:177-512
 *   - multihead_dispatch              src/common.rs:72-101
 *   - check_shapes                    src/common.rs:41-57
 *   - Kernel trait primitives         src/kernel.rs:28-98, with the scalar
 *     (src/scalar.rs:44-132), AVX2+FMA (src/avx2.rs) and AVX-512F
 *     (src/avx512.rs) implementations, selected at runtime like
 *     src/v2.rs:63-77 (AVX-512F, then AVX2+FMA, then scalar; the SSE4.1
 *     tier is not restated -- every host this runs on has AVX2).
 *
 * Pinning (what checks each function): see the header comment of
 * fa_oracle.c and tests/test_oracle.py.
 */
#ifndef FA_ORACLE_H
#define FA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Kernel tiers (src/v2.rs:63-120 picks the best available at runtime). */
enum { ORACLE_TIER_AUTO = -1, ORACLE_TIER_SCALAR = 0, ORACLE_TIER_AVX2 = 1, ORACLE_TIER_AVX512 = 2 };

/* Variants. */
enum { ORACLE_V1 = 1, ORACLE_V2 = 2, ORACLE_V3 = 3 };

/* Best tier this CPU supports (what the reference's dispatch would pick). */
int oracle_best_tier(void);
/* 1 if `tier` can run on this CPU. */
int oracle_tier_available(int tier);

/*
 * One tiled run over `bh` independent (batch*head) slices, laid out
 * [bh, seq, d] contiguous.  block sizes are clamped exactly like
 * src/v2.rs:172-173.  Zero-sized dims return without touching `out`
 * (src/common.rs:56).  `nthreads` = 0 uses every online CPU.  Returns 0, or
 * -1 for an unknown variant/tier.
 */
int oracle_run(int variant, int tier, int nthreads,
               const float* q, const float* k, const float* v,
               size_t bh, size_t seq_q, size_t seq_k, size_t d_head,
               size_t block_q, size_t block_kv, int causal, float* out);

/* Single-head, f32 restatement of naive_attention (src/naive.rs:14-75). */
void oracle_naive_f32(const float* q, const float* k, const float* v,
                      size_t seq_q, size_t seq_k, size_t d_head, int causal, float* out);

/* Same math carried out entirely in double precision (the math oracle). */
void oracle_naive_f64(const float* q, const float* k, const float* v,
                      size_t seq_q, size_t seq_k, size_t d_head, int causal, double* out);

/* Rows [row0, row0+nrows) of the double-precision naive result, for
 * spot-checking long sequences without an O(seq_q*seq_k) score matrix. */
void oracle_naive_f64_rows(const float* q, const float* k, const float* v,
                           size_t seq_q, size_t seq_k, size_t d_head, int causal,
                           size_t row0, size_t nrows, double* out);

/* The vectorised exp of the SIMD tiers (src/avx512.rs:244-291), applied
 * lane-wise; n need not be a multiple of the vector width. */
void oracle_exp_simd(int tier, const float* x, float* y, size_t n);

/* Kernel primitives exposed for unit tests (src/kernel.rs:28-98). */
float oracle_k_dot(int tier, const float* a, const float* b, size_t n);
void oracle_k_dot4x4(int tier, const float* q /*4 rows x d*/, const float* k /*4 rows x d*/,
                     size_t d, float* out /*4x4*/);
void oracle_k_pv4(int tier, float* acc /*4 rows x d*/, const float* v /*bc x d*/,
                  const float* p /*4 rows x bc*/, size_t bc, size_t d);
float oracle_k_max_reduce(int tier, const float* x, size_t n);
float oracle_k_sub_exp_sum(int tier, float* x, size_t n, float m);

/* Planted mistakes for the oracle's own pinning tests.  0 restores the
 * faithful restatement.  Not thread-safe against concurrent oracle_run. */
enum {
    ORACLE_MUTANT_NONE = 0,
    ORACLE_MUTANT_NO_CORRECTION = 1,  /* online-softmax correction dropped   */
    ORACLE_MUTANT_MASK_DIAGONAL = 2,  /* causal cutoff one key too early     */
    ORACLE_MUTANT_SCALE_1_OVER_D = 3, /* 1/d instead of 1/sqrt(d)            */
    ORACLE_MUTANT_V_SHIFT = 4         /* PV reads V rows shifted by one      */
};
void oracle_set_mutant(int which);

#ifdef __cplusplus
}
#endif
#endif
