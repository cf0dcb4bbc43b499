/*
 * fa_oracle.c -- CPU restatement of the reference crate's attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  The parity checker for the HIP kernels and the
 * timed CPU baseline ("port") in bench.py.  Nothing in the product links or
 * loads this file's library.
 *
 * Restated functions (reference = amaye15/flash-attention-cpu):
 *   tile_v2       run_v2's per-query-block body        src/v2.rs:190-383
 *   tile_v1       run_v1's per-query-block body        src/v1.rs:190-394
 *   tile_v3       run_v3 + compute_tile + finish_tile  src/v3.rs:177-348, 395-510
 *   oracle_run    par_chunks_mut over query blocks     src/v2.rs:175
 *                 + multihead_dispatch over (b,h)      src/common.rs:72-101
 *   scalar ops    ScalarKernel                         src/scalar.rs:44-132
 *   naive         naive_attention                      src/naive.rs:14-75
 *
 * Pinning (tests/test_oracle.py):
 *   - every variant and tier vs oracle_naive_f64 (double-precision textbook
 *     attention) and vs an independent numpy float64 attention, on the shape
 *     matrix of tests/correctness.rs, to 1e-3 max-abs (the reference's bar,
 *     tests/correctness.rs:109) and in practice ~1e-6;
 *   - known answers: causal row 0 == V[0] (tests/correctness.rs:240-263);
 *     seq_k == 1 => every row == V[0]; Q == 0 => each row is the mean of its
 *     visible V rows; permuting K/V rows together leaves non-causal output
 *     unchanged; adding the same vector to every K row shifts each row's
 *     scores by a constant and leaves the output unchanged;
 *   - v2 and v3 are bit-identical (same arithmetic per row, src/v3.rs);
 *     v1 agrees with v2 to 1e-5;
 *   - block-size independence incl. block 0 clamp (tests/correctness.rs:510-537);
 *   - zero-sized dims leave `out` untouched (tests/correctness.rs:465-504);
 *   - the SIMD exp vs libm expf, rel < 1e-5 on [-80, 80) step 0.1
 *     (src/avx512.rs:596-623), and each SIMD primitive vs the scalar one;
 *   - committed golden vectors (tests/golden/) computed by numpy float64.
 *   Planted-mistake tests switch on one deliberate bug at a time with
 *   oracle_set_mutant() (dropped correction, diagonal masked, 1/d scale,
 *   V rows shifted by one) and check that the pins above catch each one.
 */
#include "fa_oracle.h"
#include "fa_kernel_ops.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---------------------------------------------------------------------------
 * Scalar tier (src/scalar.rs:44-132).  Compiled with -ffp-contract=off so
 * `a*b + c` rounds twice, as Rust evaluates it.
 * ------------------------------------------------------------------------- */
static float s_dot(const float* a, const float* b, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}
static void s_dot4(const float* a0, const float* a1, const float* a2, const float* a3, const float* b,
                   size_t n, float out[4]) {
    out[0] = s_dot(a0, b, n);
    out[1] = s_dot(a1, b, n);
    out[2] = s_dot(a2, b, n);
    out[3] = s_dot(a3, b, n);
}
static void s_dot4x4(const float* const q[4], const float* const k[4], size_t n, float out[4][4]) {
    for (int r = 0; r < 4; ++r)
        for (int c = 0; c < 4; ++c) out[r][c] = s_dot(q[r], k[c], n);
}
static float s_sub_exp_sum(float* x, size_t n, float m) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - m);
        sum += x[i];
    }
    return sum;
}
static void s_axpy(float* dst, const float* src, size_t n, float s) {
    for (size_t i = 0; i < n; ++i) dst[i] += src[i] * s;
}
static void s_pv4(float* const acc[4], const float* v, const float* const p[4], size_t bc, size_t d) {
    for (size_t j = 0; j < bc; ++j)
        for (int r = 0; r < 4; ++r) s_axpy(acc[r], v + j * d, d, p[r][j]);
}
static void s_scale(float* dst, size_t n, float s) {
    for (size_t i = 0; i < n; ++i) dst[i] *= s;
}
static float s_max_reduce(const float* x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; ++i) m = fmaxf(m, x[i]);
    return m;
}
static void s_max_reduce4(const float* const x[4], size_t n, float out[4]) {
    for (int r = 0; r < 4; ++r) out[r] = s_max_reduce(x[r], n);
}
static void s_sub_exp_sum4(float* const x[4], size_t n, const float m[4], float out[4]) {
    for (int r = 0; r < 4; ++r) out[r] = s_sub_exp_sum(x[r], n, m[r]);
}
static void s_exp_vec(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

const fa_kernel_ops fa_ops_scalar = {
    s_dot, s_dot4, s_dot4x4, s_sub_exp_sum, s_axpy, s_pv4, s_scale,
    s_max_reduce, s_max_reduce4, s_sub_exp_sum4, s_exp_vec,
};

/* ---------------------------------------------------------------------------
 * Tier selection (src/v2.rs:63-120).
 * ------------------------------------------------------------------------- */
int oracle_tier_available(int tier) {
    switch (tier) {
        case ORACLE_TIER_SCALAR: return 1;
        case ORACLE_TIER_AVX2: return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
        case ORACLE_TIER_AVX512: return __builtin_cpu_supports("avx512f");
        default: return 0;
    }
}
int oracle_best_tier(void) {
    if (oracle_tier_available(ORACLE_TIER_AVX512)) return ORACLE_TIER_AVX512;
    if (oracle_tier_available(ORACLE_TIER_AVX2)) return ORACLE_TIER_AVX2;
    return ORACLE_TIER_SCALAR;
}
static const fa_kernel_ops* ops_for(int tier) {
    if (tier == ORACLE_TIER_AUTO) tier = oracle_best_tier();
    if (!oracle_tier_available(tier)) return NULL;
    switch (tier) {
        case ORACLE_TIER_SCALAR: return &fa_ops_scalar;
        case ORACLE_TIER_AVX2: return &fa_ops_avx2;
        case ORACLE_TIER_AVX512: return &fa_ops_avx512;
        default: return NULL;
    }
}

/* ---------------------------------------------------------------------------
 * Shared tile pieces.
 * ------------------------------------------------------------------------- */
typedef struct {
    const fa_kernel_ops* K;
    const float *q, *k, *v;
    size_t seq_q, seq_k, d, br, bc;
    int causal;
    float scale;
    float* out;
} head_ctx;

typedef struct {
    float *m, *l, *acc, *s0, *s1;
} scratch_t;

/* Planted-mistake switch for the pinning tests (0 = the faithful oracle). */
static int g_mutant = 0;
void oracle_set_mutant(int which) { g_mutant = which; }

/* S = scale * Q_blk K_tile^T with the 4x4 / dot4 / dot blocking, then the
 * diagonal-tile causal mask (src/v2.rs:218-287, src/v3.rs:177-257). */
static void compute_scores(const head_ctx* c, const float* q_block, size_t this_br, size_t q_start,
                           size_t k_start, size_t this_bc, float* s) {
    const fa_kernel_ops* K = c->K;
    const size_t d = c->d;
    const float* k_block = c->k + k_start * d;
    size_t i = 0;
    for (; i + 4 <= this_br; i += 4) {
        const float* qg[4] = {q_block + i * d, q_block + (i + 1) * d, q_block + (i + 2) * d,
                              q_block + (i + 3) * d};
        size_t j = 0;
        for (; j + 4 <= this_bc; j += 4) {
            const float* kg[4] = {k_block + j * d, k_block + (j + 1) * d, k_block + (j + 2) * d,
                                  k_block + (j + 3) * d};
            float t[4][4];
            K->dot4x4(qg, kg, d, t);
            for (int r = 0; r < 4; ++r)
                for (int cc = 0; cc < 4; ++cc) s[(i + r) * this_bc + j + cc] = t[r][cc] * c->scale;
        }
        for (; j < this_bc; ++j) {
            float t[4];
            K->dot4(qg[0], qg[1], qg[2], qg[3], k_block + j * d, d, t);
            for (int r = 0; r < 4; ++r) s[(i + r) * this_bc + j] = t[r] * c->scale;
        }
    }
    for (; i < this_br; ++i)
        for (size_t j = 0; j < this_bc; ++j)
            s[i * this_bc + j] = K->dot(q_block + i * d, k_block + j * d, d) * c->scale;

    if (c->causal && k_start + this_bc - 1 > q_start) {
        for (size_t r = 0; r < this_br; ++r) {
            size_t gi = q_start + r;
            size_t cutoff = (gi + 1 >= k_start) ? (gi + 1 - k_start) : 0;
            if (g_mutant == ORACLE_MUTANT_MASK_DIAGONAL && cutoff > 0) cutoff -= 1;
            if (cutoff > this_bc) cutoff = this_bc;
            for (size_t j = cutoff; j < this_bc; ++j) s[r * this_bc + j] = -INFINITY;
        }
    }
}

/* Online-softmax update + PV for one tile (v2/v3: deferred normalisation,
 * src/v2.rs:289-372, src/v3.rs:267-348).  v1 == 1 applies v1's per-step
 * un-normalise / re-normalise instead (src/v1.rs:291-385). */
static void finish_scores(const head_ctx* c, float* s, size_t this_br, size_t k_start, size_t this_bc,
                          float* m, float* l, float* acc, int v1) {
    const fa_kernel_ops* K = c->K;
    const size_t d = c->d;
    const float* v_block = c->v + k_start * d;
    if (g_mutant == ORACLE_MUTANT_V_SHIFT && k_start + this_bc < c->seq_k) v_block += d;
    size_t i = 0;
    for (; i + 4 <= this_br; i += 4) {
        const float* rows_c[4] = {s + i * this_bc, s + (i + 1) * this_bc, s + (i + 2) * this_bc,
                                  s + (i + 3) * this_bc};
        float* rows[4] = {s + i * this_bc, s + (i + 1) * this_bc, s + (i + 2) * this_bc,
                          s + (i + 3) * this_bc};
        float bmax[4], new_m[4], bsum[4];
        K->max_reduce4(rows_c, this_bc, bmax);
        for (int r = 0; r < 4; ++r) new_m[r] = fmaxf(m[i + r], bmax[r]);
        K->sub_exp_sum4(rows, this_bc, new_m, bsum);
        for (int r = 0; r < 4; ++r) {
            float corr = expf(m[i + r] - new_m[r]);
            if (g_mutant == ORACLE_MUTANT_NO_CORRECTION) corr = 1.0f;
            if (v1) {
                float old_l = l[i + r];
                float new_l = corr * old_l + bsum[r];
                K->scale(acc + (i + r) * d, d, old_l * corr);
                m[i + r] = new_m[r];
                l[i + r] = new_l;
            } else {
                l[i + r] = corr * l[i + r] + bsum[r];
                K->scale(acc + (i + r) * d, d, corr);
                m[i + r] = new_m[r];
            }
        }
    }
    for (; i < this_br; ++i) {
        float* row = s + i * this_bc;
        float bmax = K->max_reduce(row, this_bc);
        float new_m = fmaxf(m[i], bmax);
        float bsum = K->sub_exp_sum(row, this_bc, new_m);
        float corr = expf(m[i] - new_m);
        if (g_mutant == ORACLE_MUTANT_NO_CORRECTION) corr = 1.0f;
        if (v1) {
            float old_l = l[i];
            float new_l = corr * old_l + bsum;
            K->scale(acc + i * d, d, old_l * corr);
            m[i] = new_m;
            l[i] = new_l;
        } else {
            l[i] = corr * l[i] + bsum;
            K->scale(acc + i * d, d, corr);
            m[i] = new_m;
        }
    }

    i = 0;
    for (; i + 4 <= this_br; i += 4) {
        float* a[4] = {acc + i * d, acc + (i + 1) * d, acc + (i + 2) * d, acc + (i + 3) * d};
        const float* p[4] = {s + i * this_bc, s + (i + 1) * this_bc, s + (i + 2) * this_bc,
                             s + (i + 3) * this_bc};
        K->pv4(a, v_block, p, this_bc, d);
    }
    for (; i < this_br; ++i)
        for (size_t j = 0; j < this_bc; ++j) K->axpy(acc + i * d, v_block + j * d, d, s[i * this_bc + j]);

    if (v1) {
        for (size_t r = 0; r < this_br; ++r) {
            float inv = l[r] > 0.0f ? 1.0f / l[r] : 0.0f;
            K->scale(acc + r * d, d, inv);
        }
    }
}

static void reset_state(size_t this_br, size_t d, float* m, float* l, float* acc) {
    for (size_t r = 0; r < this_br; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
    }
    memset(acc, 0, this_br * d * sizeof(float));
}

static void write_normalised(size_t this_br, size_t d, const float* l, const float* acc, float* out) {
    for (size_t r = 0; r < this_br; ++r) {
        float inv = l[r] > 0.0f ? 1.0f / l[r] : 0.0f;
        for (size_t x = 0; x < d; ++x) out[r * d + x] = acc[r * d + x] * inv;
    }
}

/* run_v2 body for query block qi (src/v2.rs:190-383). */
static void tile_v2(const head_ctx* c, size_t qi, scratch_t* w) {
    const size_t d = c->d, br = c->br, bc = c->bc;
    const size_t q_start = qi * br;
    const size_t this_br = (c->seq_q - q_start < br) ? c->seq_q - q_start : br;
    const float* q_block = c->q + q_start * d;
    reset_state(this_br, d, w->m, w->l, w->acc);
    const size_t nkv = (c->seq_k + bc - 1) / bc;
    for (size_t kj = 0; kj < nkv; ++kj) {
        size_t k_start = kj * bc;
        size_t this_bc = (c->seq_k - k_start < bc) ? c->seq_k - k_start : bc;
        if (c->causal && k_start > q_start + this_br - 1) break;
        compute_scores(c, q_block, this_br, q_start, k_start, this_bc, w->s0);
        finish_scores(c, w->s0, this_br, k_start, this_bc, w->m, w->l, w->acc, 0);
    }
    write_normalised(this_br, d, w->l, w->acc, c->out + q_start * d);
}

/* run_v1 body (src/v1.rs:190-394): no causal break, acc kept normalised. */
static void tile_v1(const head_ctx* c, size_t qi, scratch_t* w) {
    const size_t d = c->d, br = c->br, bc = c->bc;
    const size_t q_start = qi * br;
    const size_t this_br = (c->seq_q - q_start < br) ? c->seq_q - q_start : br;
    const float* q_block = c->q + q_start * d;
    reset_state(this_br, d, w->m, w->l, w->acc);
    const size_t nkv = (c->seq_k + bc - 1) / bc;
    for (size_t kj = 0; kj < nkv; ++kj) {
        size_t k_start = kj * bc;
        size_t this_bc = (c->seq_k - k_start < bc) ? c->seq_k - k_start : bc;
        compute_scores(c, q_block, this_br, q_start, k_start, this_bc, w->s0);
        finish_scores(c, w->s0, this_br, k_start, this_bc, w->m, w->l, w->acc, 1);
    }
    memcpy(c->out + q_start * d, w->acc, this_br * d * sizeof(float));
}

/* run_v3 body (src/v3.rs:395-510): last_kj hoisted, tile kj+1's scores
 * computed into the other buffer before tile kj is finished. */
static void tile_v3(const head_ctx* c, size_t qi, scratch_t* w) {
    const size_t d = c->d, br = c->br, bc = c->bc;
    const size_t q_start = qi * br;
    const size_t this_br = (c->seq_q - q_start < br) ? c->seq_q - q_start : br;
    const float* q_block = c->q + q_start * d;
    float* out = c->out + q_start * d;
    reset_state(this_br, d, w->m, w->l, w->acc);
    const size_t nkv = (c->seq_k + bc - 1) / bc;
    size_t last_kj = nkv;
    if (c->causal) {
        for (size_t kj = 0; kj < nkv; ++kj)
            if (kj * bc > q_start + this_br - 1) {
                last_kj = kj;
                break;
            }
    }
    if (last_kj == 0) {
        memset(out, 0, this_br * d * sizeof(float));
        return;
    }
#define TILE_LEN(kj) ((c->seq_k - (kj) * bc < bc) ? c->seq_k - (kj) * bc : bc)
    float* buf[2] = {w->s0, w->s1};
    compute_scores(c, q_block, this_br, q_start, 0, TILE_LEN(0), buf[0]);
    for (size_t kj = 0; kj + 1 < last_kj; ++kj) {
        float* cur = buf[kj & 1];
        float* nxt = buf[(kj + 1) & 1];
        compute_scores(c, q_block, this_br, q_start, (kj + 1) * bc, TILE_LEN(kj + 1), nxt);
        finish_scores(c, cur, this_br, kj * bc, TILE_LEN(kj), w->m, w->l, w->acc, 0);
    }
    size_t last = last_kj - 1;
    finish_scores(c, buf[last & 1], this_br, last * bc, TILE_LEN(last), w->m, w->l, w->acc, 0);
#undef TILE_LEN
    write_normalised(this_br, d, w->l, w->acc, out);
}

/* ---------------------------------------------------------------------------
 * Parallel driver: tasks = (bh, query block), pulled from an atomic counter
 * by `nthreads` workers (rayon's nested par_chunks over heads and query
 * blocks, src/common.rs:92-100 and src/v2.rs:175, flattened).
 * ------------------------------------------------------------------------- */
typedef struct {
    int variant;
    head_ctx base;
    size_t bh, nqb;
    atomic_size_t next;
} job_t;

static void* worker(void* arg) {
    job_t* job = (job_t*)arg;
    const head_ctx* b = &job->base;
    size_t d = b->d;
    scratch_t w;
    w.m = (float*)malloc(b->br * sizeof(float));
    w.l = (float*)malloc(b->br * sizeof(float));
    w.acc = (float*)malloc(b->br * d * sizeof(float));
    w.s0 = (float*)malloc(b->br * b->bc * sizeof(float));
    w.s1 = (float*)malloc(b->br * b->bc * sizeof(float));
    size_t total = job->bh * job->nqb;
    for (;;) {
        size_t t = atomic_fetch_add(&job->next, 1);
        if (t >= total) break;
        size_t h = t / job->nqb, qi = t % job->nqb;
        head_ctx c = *b;
        c.q = b->q + h * b->seq_q * d;
        c.k = b->k + h * b->seq_k * d;
        c.v = b->v + h * b->seq_k * d;
        c.out = b->out + h * b->seq_q * d;
        if (job->variant == ORACLE_V1) tile_v1(&c, qi, &w);
        else if (job->variant == ORACLE_V3) tile_v3(&c, qi, &w);
        else tile_v2(&c, qi, &w);
    }
    free(w.m);
    free(w.l);
    free(w.acc);
    free(w.s0);
    free(w.s1);
    return NULL;
}

int oracle_run(int variant, int tier, int nthreads, const float* q, const float* k, const float* v,
               size_t bh, size_t seq_q, size_t seq_k, size_t d_head, size_t block_q, size_t block_kv,
               int causal, float* out) {
    if (variant != ORACLE_V1 && variant != ORACLE_V2 && variant != ORACLE_V3) return -1;
    const fa_kernel_ops* K = ops_for(tier);
    if (!K) return -1;
    if (bh == 0 || seq_q == 0 || seq_k == 0 || d_head == 0) return 0; /* src/common.rs:56 */

    job_t job;
    job.variant = variant;
    job.base.K = K;
    job.base.q = q;
    job.base.k = k;
    job.base.v = v;
    job.base.seq_q = seq_q;
    job.base.seq_k = seq_k;
    job.base.d = d_head;
    /* src/v2.rs:172-173: max(1).min(seq) */
    size_t br = block_q < 1 ? 1 : block_q;
    size_t bc = block_kv < 1 ? 1 : block_kv;
    job.base.br = br > seq_q ? seq_q : br;
    job.base.bc = bc > seq_k ? seq_k : bc;
    job.base.causal = causal != 0;
    /* src/v2.rs:171: 1.0 / (d_head as f32).sqrt() */
    job.base.scale = 1.0f / sqrtf((float)d_head);
    if (g_mutant == ORACLE_MUTANT_SCALE_1_OVER_D) job.base.scale = 1.0f / (float)d_head;
    job.base.out = out;
    job.bh = bh;
    job.nqb = (seq_q + job.base.br - 1) / job.base.br;
    atomic_init(&job.next, 0);

    long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
    int nt = nthreads > 0 ? nthreads : (int)(ncpu > 0 ? ncpu : 1);
    size_t tasks = bh * job.nqb;
    if ((size_t)nt > tasks) nt = (int)tasks;
    if (nt <= 1) {
        worker(&job);
        return 0;
    }
    pthread_t* th = (pthread_t*)malloc((size_t)nt * sizeof(pthread_t));
    int started = 0;
    for (int i = 0; i < nt; ++i)
        if (pthread_create(&th[i], NULL, worker, &job) == 0) ++started;
    if (started == 0) worker(&job);
    for (int i = 0; i < started; ++i) pthread_join(th[i], NULL);
    free(th);
    return 0;
}

/* ---------------------------------------------------------------------------
 * naive_attention (src/naive.rs:14-75), f32 and double.
 * ------------------------------------------------------------------------- */
void oracle_naive_f32(const float* q, const float* k, const float* v, size_t seq_q, size_t seq_k,
                      size_t d, int causal, float* out) {
    if (seq_q == 0 || d == 0) return;
    float scale = 1.0f / sqrtf((float)d);
    float* row = (float*)malloc((seq_k ? seq_k : 1) * sizeof(float));
    for (size_t i = 0; i < seq_q; ++i) {
        for (size_t j = 0; j < seq_k; ++j) {
            if (causal && j > i) {
                row[j] = -INFINITY;
                continue;
            }
            row[j] = s_dot(q + i * d, k + j * d, d) * scale;
        }
        float m = -INFINITY;
        for (size_t j = 0; j < seq_k; ++j) m = fmaxf(m, row[j]);
        float sum = 0.0f;
        for (size_t j = 0; j < seq_k; ++j) {
            row[j] = expf(row[j] - m);
            sum += row[j];
        }
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (size_t j = 0; j < seq_k; ++j) row[j] *= inv;
        float* o = out + i * d;
        for (size_t x = 0; x < d; ++x) o[x] = 0.0f;
        for (size_t j = 0; j < seq_k; ++j) {
            float p = row[j];
            if (p == 0.0f) continue;
            for (size_t x = 0; x < d; ++x) o[x] += p * v[j * d + x];
        }
    }
    free(row);
}

void oracle_naive_f64_rows(const float* q, const float* k, const float* v, size_t seq_q, size_t seq_k,
                           size_t d, int causal, size_t row0, size_t nrows, double* out) {
    if (d == 0 || row0 >= seq_q) return;
    if (row0 + nrows > seq_q) nrows = seq_q - row0;
    double scale = 1.0 / sqrt((double)d);
    double* row = (double*)malloc((seq_k ? seq_k : 1) * sizeof(double));
    for (size_t ii = 0; ii < nrows; ++ii) {
        size_t i = row0 + ii;
        double m = -INFINITY;
        for (size_t j = 0; j < seq_k; ++j) {
            if (causal && j > i) {
                row[j] = -INFINITY;
                continue;
            }
            double s = 0.0;
            for (size_t x = 0; x < d; ++x) s += (double)q[i * d + x] * (double)k[j * d + x];
            row[j] = s * scale;
            if (row[j] > m) m = row[j];
        }
        double sum = 0.0;
        for (size_t j = 0; j < seq_k; ++j) {
            row[j] = (row[j] == -INFINITY) ? 0.0 : exp(row[j] - m);
            sum += row[j];
        }
        double inv = sum > 0.0 ? 1.0 / sum : 0.0;
        double* o = out + ii * d;
        for (size_t x = 0; x < d; ++x) o[x] = 0.0;
        for (size_t j = 0; j < seq_k; ++j) {
            double p = row[j] * inv;
            if (p == 0.0) continue;
            for (size_t x = 0; x < d; ++x) o[x] += p * (double)v[j * d + x];
        }
    }
    free(row);
}

void oracle_naive_f64(const float* q, const float* k, const float* v, size_t seq_q, size_t seq_k,
                      size_t d, int causal, double* out) {
    oracle_naive_f64_rows(q, k, v, seq_q, seq_k, d, causal, 0, seq_q, out);
}

/* ---------------------------------------------------------------------------
 * Primitive hooks for unit tests.
 * ------------------------------------------------------------------------- */
void oracle_exp_simd(int tier, const float* x, float* y, size_t n) {
    const fa_kernel_ops* K = ops_for(tier);
    if (K) K->exp_vec(x, y, n);
}
float oracle_k_dot(int tier, const float* a, const float* b, size_t n) {
    const fa_kernel_ops* K = ops_for(tier);
    return K ? K->dot(a, b, n) : NAN;
}
void oracle_k_dot4x4(int tier, const float* q, const float* k, size_t d, float* out) {
    const fa_kernel_ops* K = ops_for(tier);
    if (!K) return;
    const float* qq[4] = {q, q + d, q + 2 * d, q + 3 * d};
    const float* kk[4] = {k, k + d, k + 2 * d, k + 3 * d};
    float t[4][4];
    K->dot4x4(qq, kk, d, t);
    for (int r = 0; r < 4; ++r)
        for (int c = 0; c < 4; ++c) out[r * 4 + c] = t[r][c];
}
void oracle_k_pv4(int tier, float* acc, const float* v, const float* p, size_t bc, size_t d) {
    const fa_kernel_ops* K = ops_for(tier);
    if (!K) return;
    float* a[4] = {acc, acc + d, acc + 2 * d, acc + 3 * d};
    const float* pp[4] = {p, p + bc, p + 2 * bc, p + 3 * bc};
    K->pv4(a, v, pp, bc, d);
}
float oracle_k_max_reduce(int tier, const float* x, size_t n) {
    const fa_kernel_ops* K = ops_for(tier);
    return K ? K->max_reduce(x, n) : NAN;
}
float oracle_k_sub_exp_sum(int tier, float* x, size_t n, float m) {
    const fa_kernel_ops* K = ops_for(tier);
    return K ? K->sub_exp_sum(x, n, m) : NAN;
}
