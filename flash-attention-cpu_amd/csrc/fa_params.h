// fa_params.h -- the one argument block every kernel in fa_kernels.hip takes.
//
// Passed by value through hipModuleLaunchKernel; the host library fills it.
// Plain C layout (pointers, then 32-bit fields) so host and device agree.
#ifndef FA_PARAMS_H
#define FA_PARAMS_H

#include <stdint.h>

typedef struct FaParams {
    const float* q;      // [bh, seq_q, d]
    const float* k;      // [bh, seq_k, d]
    const float* v;      // [bh, seq_k, d]
    float* out;          // [bh, seq_q, d]
    float* part_o;       // split-KV partial O: [bh, nqt, num_splits, 16, D]
    float* part_ml;      // split-KV partial (m, l): [bh, nqt, num_splits, 2, 16]
    int bh;              // batch * heads
    int seq_q;
    int seq_k;
    int d;               // true d_head (kernels pad to D)
    int causal;          // top-left aligned: key j visible to query i iff j <= i
    float scale_log2e;   // (1/sqrt(d) computed in f32) * log2(e)
    int nqb;             // prefill: query blocks of 128 rows
    int nqt;             // split-KV: query tiles of 16 rows
    int num_splits;      // split-KV / key split: key splits per (bh, query tile)
    int split_len;       // keys per split (split-KV: multiple of 64; key split: of the stage)
    int ks_rows;         // key split: query rows per prefill block (0: split-KV decode)
    float merge_scale;   // fa_merge: factor taking partial maxima to the log2 domain
                         // (split-KV: scale_log2e; prefill key split: 1, already scaled)
    int pair_w;          // prefill, two workgroups per CU: causal ranks per dispatch round
                         // (odd rounds run in reverse so each CU pairs a long and a short
                         // block); 0 = plain longest-first order
    int two_blocks;      // f32 v3 prefill, d_head 128: each workgroup runs query blocks
                         // nqb-1-r and r of one (batch, head); nqb even, grid = bh * nqb / 2
    int full_keys;       // v1: every query block visits all seq_k keys, causal or not (no
                         // causal skip), so the key split, the stream split and fa_merge
                         // count each block's keys as the whole key range
    long long stream_per;         // stream split (v2/v3 prefill): key stages per workgroup; 0 = off
    long long stream_head_units;  // stream split: key stages of one slice (all its query blocks)
} FaParams;


// Naive attention (materialised scores): one chunk of heads per launch.
typedef struct NaiveParams {
    const float* q;      // [heads, seq_q, d] (this chunk)
    const float* k;      // [heads, seq_k, d]
    const float* v;      // [heads, seq_k, d]
    float* out;          // [heads, seq_q, d]
    void* s;             // scores / probabilities [heads, seq_q, seq_k], f32 or f64
    int seq_q;
    int seq_k;
    int d;
    int causal;
    float scale_f;       // 1/sqrt(d) in f32 (src/naive.rs:29)
    double scale_d;      // 1/sqrt(d) in f64 (f64 instantiation)
} NaiveParams;

// Peak probes (fa_probe_mfma_*, fa_probe_copy): the machine's own ceilings
// for the roofline denominators.
typedef struct ProbeParams {
    float* buf;                 // MFMA probes: one checksum per wave; copy: source half, then destination half
    unsigned long long n16;     // copy: 16-byte elements per half
    unsigned iters;             // MFMA probes: iterations of the independent MFMA chains
} ProbeParams;


// Prefill geometry shared by the host planner and the kernels: waves per
// workgroup (each wave owns 16 query rows) and keys per LDS stage.
// FA_PREFILL_WAVES selects the workgroup size for d_head <= 128.
#ifndef FA_PREFILL_WAVES
#define FA_PREFILL_WAVES 8
#endif
// fa_merge: output rows per workgroup (one wave each).
#define FA_MERGE_ROWS 4
#ifdef __cplusplus
constexpr int fa_prefill_waves(int D) { return D <= 128 ? FA_PREFILL_WAVES : 8; }
// d_head > 256 (D = 512, 1024): column groups of D / 256 waves share each
// 16-row tile, every wave holding 256 columns of Q and O.
constexpr int fa_prefill_cgroups(int D) { return D > 256 ? D / 256 : 1; }
constexpr int fa_prefill_rows(int D) { return 16 * fa_prefill_waves(D) / fa_prefill_cgroups(D); }
// d = 256: v3 keeps two stages resident and fits its registers only with
// 16-key stages; v1/v2 (one stage) use 32.  D > 256: 16-key stages.
// Low-precision (bf16 / f16) prefill: 128-row workgroups of waves owning MT
// 16-row tiles each (MT = 1, or 2 for D = 128); 64-key stages.
constexpr int fa_lp_rows() { return 128; }
constexpr int fa_lp_waves(int MT) { return fa_lp_rows() / (16 * MT); }
constexpr int fa_lp_stage_keys() { return 64; }
constexpr int fa_prefill_stage_keys(int D, int variant) {
    return D <= 128 ? (fa_prefill_waves(D) == 8 ? 64 : 32) : (D > 256 || variant == 3 ? 16 : 32);
}
// D = 1024: one 16-key stage of K and V takes 130 KiB of LDS, so v3 keeps a
// single stage (its math is v2's; only the double-buffered schedule goes).
constexpr int fa_prefill_nbuf(int D, int variant) { return variant == 3 && D <= 512 ? 2 : 1; }
// v3 fills its LDS stages by global->LDS DMA (loader 2) up to D = 1024 (two
// stages up to 512, alternating K / V buffers at 1024); D = 2048 keeps one
// K-or-V buffer filled through registers for every variant.
constexpr bool fa_prefill_dma(int D, int variant) { return variant == 3 && D <= 1024; }
#endif

#endif
