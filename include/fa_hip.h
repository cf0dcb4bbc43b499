/*
 * fa_hip.h -- C ABI of the MI355X FlashAttention library (libfa_hip.so).
 *
 * The drop-in boundary for the reference crate amaye15/flash-attention-cpu:
 * every entry point below replaces one public Rust function of that crate
 * (cited per declaration) with the same argument meaning: row-major f32
 * Q/K/V/O, [batch, heads, seq, d_head] for the multi-head forms, the causal
 * flag of FlashAttentionConfig, and the implicit softmax scale
 * 1/sqrt(d_head) computed in f32.  Rust slices become (pointer, length)
 * pairs so the crate's shape asserts keep their meaning; a failed assert
 * becomes a non-zero status instead of a panic, naming the same operand.
 *
 * All compute runs on the GPU (hand-written gfx950 kernels loaded from a
 * code object with hipModuleLoad); there is no CPU fallback.  Host-slice
 * entry points copy to device memory, launch, copy back and synchronise;
 * the _device forms take caller-owned device pointers and the caller's HIP
 * stream and return as soon as the kernels are queued.
 *
 * Thread safety: every entry point may be called from several threads at
 * once (the crate's functions are Sync).  Up to four host-slice calls per
 * device run concurrently, each on its own stream, device staging buffer and
 * pinned copy ring; further callers wait until one of those four finishes.
 */
#ifndef FA_HIP_H
#define FA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define FA_OK 0
#define FA_ERR_Q_SHAPE 1      /* "q shape mismatch"   src/common.rs:51, :87 */
#define FA_ERR_K_SHAPE 2      /* "k shape mismatch"   src/common.rs:52, :88 */
#define FA_ERR_V_SHAPE 3      /* "v shape mismatch"   src/common.rs:53, :89 */
#define FA_ERR_OUT_SHAPE 4    /* "out shape mismatch" src/common.rs:54, :90 */
#define FA_ERR_INVALID_ARG 5  /* NULL pointer with a non-zero length, bad variant/option */
#define FA_ERR_UNSUPPORTED 6  /* d_head > 256 with 16-bit inputs or a forced split-KV path,
                                 d_head > 2048 with a forced stream split or a split count, or a
                                 size beyond 32-bit row indexing (f32 heads of any width run the
                                 flash kernels) */
#define FA_ERR_NO_DEVICE 7    /* no HIP device visible */
#define FA_ERR_MODULE 8       /* code object missing / unloadable (FA_HIP_MODULE) */
#define FA_ERR_ALLOC 9        /* device allocation failed, or the request exceeds the free
                                 device memory (checked before anything is queued) */
#define FA_ERR_LAUNCH 10      /* kernel launch failed */
#define FA_ERR_COPY 11        /* host<->device copy or synchronisation failed */
#define FA_ERR_SCRATCH 12     /* fa_device_ex_noalloc: the call needs more split workspace than
                                 the 64 MiB scratch array, or the array is unavailable */

/* Human-readable text for a status code (static storage). */
const char* fa_status_string(int status);

/* ---- configuration ------------------------------------------------------
 * Mirrors FlashAttentionConfig (src/common.rs:16-36).  block_size_q and
 * block_size_kv are accepted for signature parity; the GPU tiles are fixed
 * per d_head and results do not depend on block sizes beyond rounding, as
 * in the reference (tests/correctness.rs:137-171).  causal: key j is
 * visible to query i iff j <= i, in absolute indices (src/naive.rs:37). */
typedef struct fa_config {
    size_t block_size_q;   /* default 64  */
    size_t block_size_kv;  /* default 128 */
    uint8_t causal;        /* default 0   */
} fa_config;

/* FlashAttentionConfig::default() -- src/common.rs:28-36 */
fa_config fa_config_default(void);

/* ---- single head, host slices ------------------------------------------
 * q: [seq_len_q, d_head], k/v: [seq_len_k, d_head], out: [seq_len_q, d_head].
 * Checks q/k/v/out lengths in that order (check_shapes, src/common.rs:41-57);
 * if seq_len_q, seq_len_k or d_head is 0 returns FA_OK without touching out.
 * config == NULL means fa_config_default(). */

/* flash_attention_v1 -- src/v1.rs:51-123 (FA-1: per-step normalisation,
 * no causal tile skip) */
int fa_v1(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
          size_t seq_len_q, size_t seq_len_k, size_t d_head, const fa_config* config, float* out,
          size_t out_len);
/* flash_attention_v2 -- src/v2.rs:49-121 (FA-2: deferred normalisation,
 * causal skip of fully-future tiles) */
int fa_v2(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
          size_t seq_len_q, size_t seq_len_k, size_t d_head, const fa_config* config, float* out,
          size_t out_len);
/* flash_attention_v3 -- src/v3.rs:61-133 (v2 with the next tile's QK^T
 * overlapped with the current softmax + PV) */
int fa_v3(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
          size_t seq_len_q, size_t seq_len_k, size_t d_head, const fa_config* config, float* out,
          size_t out_len);
/* flash_attention (alias of v2) -- src/lib.rs:87 */
int fa_attention(const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                 size_t v_len, size_t seq_len_q, size_t seq_len_k, size_t d_head,
                 const fa_config* config, float* out, size_t out_len);

/* ---- batched multi-head, host slices ----------------------------------
 * q/out: [batch, heads, seq_len_q, d_head], k/v: [batch, heads, seq_len_k,
 * d_head], contiguous (multihead_dispatch, src/common.rs:72-101).  All
 * batch*heads slices run in one launch. */

/* flash_attention_multihead_v1 -- src/v1.rs:134-159 */
int fa_multihead_v1(const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                    size_t v_len, size_t batch, size_t heads, size_t seq_len_q, size_t seq_len_k,
                    size_t d_head, const fa_config* config, float* out, size_t out_len);
/* flash_attention_multihead_v2 -- src/v2.rs:132-157 */
int fa_multihead_v2(const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                    size_t v_len, size_t batch, size_t heads, size_t seq_len_q, size_t seq_len_k,
                    size_t d_head, const fa_config* config, float* out, size_t out_len);
/* flash_attention_multihead_v3 -- src/v3.rs:144-169 */
int fa_multihead_v3(const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                    size_t v_len, size_t batch, size_t heads, size_t seq_len_q, size_t seq_len_k,
                    size_t d_head, const fa_config* config, float* out, size_t out_len);
/* flash_attention_multihead (alias of multihead v2) -- src/lib.rs:86 */
int fa_attention_multihead(const float* q, size_t q_len, const float* k, size_t k_len,
                           const float* v, size_t v_len, size_t batch, size_t heads,
                           size_t seq_len_q, size_t seq_len_k, size_t d_head,
                           const fa_config* config, float* out, size_t out_len);

/* ---- device-resident, stream-ordered -----------------------------------
 * Same computation as fa_multihead_vN on device pointers (hipMalloc'd or any
 * device-accessible memory), queued on `stream` (a hipStream_t; NULL = the
 * default stream).  No length checks are possible on raw pointers; zero
 * dims return FA_OK with nothing queued.  Every variant picks the split-KV
 * (flash-decoding) kernels for short query blocks against long key ranges,
 * and a key or stream split on grids smaller than the GPU (v1 on kernels of
 * its own that keep its per-step normalisation and visit every key, causal
 * or not).  Their partials go to a
 * workspace kept per stream (up to 256 MiB; larger ones are allocated and
 * released stream-ordered around the call): the first call on a stream that
 * needs more allocates it with hipMalloc, and buffers are kept (outgrown ones
 * included) until fa_release_stream_workspace or the end of the process, so
 * graphs captured with these calls stay valid.  A call made under graph
 * capture takes the stream's buffer over for the graph (make one eager call
 * on the stream before each capture; the next eager call allocates anew), so
 * replays never share partials with other calls.  Calls on one stream share
 * its buffer in stream order; a stream handle value reused after
 * hipStreamDestroy inherits the buffer, so release a stream's workspace (or
 * synchronise it) before destroying it if its handle may be reused.
 * These have no single counterpart in the reference (its API takes host
 * slices); they are the device form of the multihead entry points. */
int fa_device_v1(void* stream, const float* q, const float* k, const float* v, size_t batch,
                 size_t heads, size_t seq_len_q, size_t seq_len_k, size_t d_head,
                 const fa_config* config, float* out);
int fa_device_v2(void* stream, const float* q, const float* k, const float* v, size_t batch,
                 size_t heads, size_t seq_len_q, size_t seq_len_k, size_t d_head,
                 const fa_config* config, float* out);
int fa_device_v3(void* stream, const float* q, const float* k, const float* v, size_t batch,
                 size_t heads, size_t seq_len_q, size_t seq_len_k, size_t d_head,
                 const fa_config* config, float* out);
/* Frees the split workspace kept for `stream` on the current device (and the
 * buffers it outgrew), after synchronising the stream.  For servers that
 * create and destroy streams: call it before hipStreamDestroy.  Graphs
 * captured with split calls on `stream` must not be replayed afterwards.  A
 * later split call on the stream allocates a new workspace.  No counterpart
 * in the reference (the crate's scratch is per call). */
int fa_release_stream_workspace(void* stream);

/* ---- extension: explicit scale and path control ------------------------
 * Not in the reference.  softmax_scale <= 0 or NaN keeps the reference's
 * 1/sqrt(d_head).  path: FA_PATH_AUTO (what fa_device_vN does),
 * FA_PATH_PREFILL (query-block kernel; with num_splits > 1, each block's
 * keys are divided over num_splits workgroups whose partials are merged),
 * FA_PATH_SPLITKV (16-row decode tiles; with one split -- num_splits = 1, or
 * chosen -- each tile is written directly, no merge), FA_PATH_SPLITKV_ROWS
 * (row-streaming split-KV for seq_len_q <= 4: K and V read as whole rows,
 * dot products on the vector ALUs; f32, d_head % 4 == 0 and 16-byte aligned
 * operands, else FA_ERR_UNSUPPORTED), FA_PATH_STREAM (query-block kernel
 * with the stream split: the key stages of every (slice, query block) cut
 * into equal runs, one per workgroup -- num_splits workgroups, 0 = one per
 * resident workgroup slot -- with partials merged where a block is shared).
 * Every path takes every variant; v1's split kernels keep its per-step
 * normalisation and visit every key (no causal skip).  AUTO runs
 * decode steps -- seq_len_q <= 32, any batch and key count -- on split-KV
 * (the row-streaming kernel where it applies, else 16-row tiles; 16-bit
 * inputs only on the row kernel), and the stream split or the key split for
 * prefills smaller than the GPU.
 * num_splits = 0 lets the library choose (at most 1024). */
#define FA_PATH_AUTO 0
#define FA_PATH_PREFILL 1
#define FA_PATH_SPLITKV 2
#define FA_PATH_SPLITKV_ROWS 3
#define FA_PATH_STREAM 4
/* Element type of Q, K, V (O is always f32). */
#define FA_DTYPE_F32 0
#define FA_DTYPE_BF16 1
#define FA_DTYPE_F16 2
typedef struct fa_launch_opts {
    float softmax_scale;
    int path;
    int num_splits;
    int dtype;   /* FA_DTYPE_*: read by fa_describe_launch; fa_device_ex accepts only F32 */
} fa_launch_opts;

int fa_device_ex(int variant, void* stream, const float* q, const float* k, const float* v,
                 size_t batch, size_t heads, size_t seq_len_q, size_t seq_len_k, size_t d_head,
                 const fa_config* config, const fa_launch_opts* opts, float* out);

/* ---- allocation-free form ------------------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  Same arguments, kernels and results as fa_device_ex,
 * but the split partials (split-KV decode, prefill key split) go to a
 * device-global scratch array of 64 MiB per GPU, held until the process
 * ends, and the call allocates and frees nothing.  Calls whose plan needs a
 * larger workspace return FA_ERR_SCRATCH (out untouched).  Call fa_init()
 * on each device first (it loads the kernels and maps the array; a first
 * call does it itself, which allocates).  All calls on one GPU share its
 * array: calls that may overlap on one GPU (different streams, or graphs
 * replayed concurrently) race on it and must be ordered by the caller. */
int fa_device_ex_noalloc(int variant, void* stream, const float* q, const float* k, const float* v,
                         size_t batch, size_t heads, size_t seq_len_q, size_t seq_len_k, size_t d_head,
                         const fa_config* config, const fa_launch_opts* opts, float* out);

/* ---- 16-bit inputs (bf16 / f16) -------------------------------------------
 * Not in the reference, whose roadmap plans bf16 dot products with f32
 * accumulation (ROADMAP.md, item 2 "bf16 dot-product acceleration").  Q, K, V
 * hold bfloat16 (FA_DTYPE_BF16, raw 16-bit patterns) or IEEE binary16
 * (FA_DTYPE_F16) in the layout of the f32 entry points; O is f32.  QK^T and PV
 * run on 16-bit MFMA with f32 accumulation (every product exact), the softmax
 * in f32, and the probabilities are rounded to the input type for PV (the
 * row sums add up the rounded values), so each output element is within
 * u/(1-u) * max|V| of f32 attention on the same 16-bit inputs (u = 2^-8
 * bf16, 2^-11 f16; f16 probabilities are rounded as 2^7 p, so only those
 * below 2^-21 of the row's reference fall below f16's normal range, adding
 * at most n * 2^-32 * max|V| over a row of n keys).  Causal masking, shape checks and
 * zero-dimension behaviour are those of fa_multihead_v2; d_head <= 256.  The
 * algorithm is v2/v3's (deferred normalisation, causal skip); no variant
 * argument.  opts: softmax_scale, path and num_splits as for fa_device_ex;
 * opts->dtype is ignored.  The split-KV kernels (FA_PATH_SPLITKV, and
 * FA_PATH_SPLITKV_ROWS for seq_len_q = 1, d_head % 8 == 0, d_head > 32, which
 * AUTO picks for decode steps) widen the 16-bit values exactly and compute in
 * f32 without rounding the probabilities. */
int fa_device_lp(int dtype, void* stream, const void* q, const void* k, const void* v, size_t batch,
                 size_t heads, size_t seq_len_q, size_t seq_len_k, size_t d_head,
                 const fa_config* config, const fa_launch_opts* opts, float* out);
/* Host-slice form; lengths count elements. */
int fa_multihead_lp(int dtype, const void* q, size_t q_len, const void* k, size_t k_len,
                    const void* v, size_t v_len, size_t batch, size_t heads, size_t seq_len_q,
                    size_t seq_len_k, size_t d_head, const fa_config* config, float* out,
                    size_t out_len);

/* ---- naive attention (materialised scores) -------------------------------
 * naive_attention -- src/naive.rs:14-75: the textbook O(seq_q * seq_k)
 * memory form (scores, row softmax, PV) that the crate keeps as its
 * correctness oracle, here on the GPU.  Same shape checks and order
 * (src/naive.rs:24-27); seq_len_q or d_head == 0 writes nothing, seq_len_k
 * == 0 writes zeros (the crate's out_row.fill).  f32 arithmetic. */
int fa_naive_attention(const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                       size_t v_len, size_t seq_len_q, size_t seq_len_k, size_t d_head, int causal,
                       float* out, size_t out_len);
/* Device-resident, multi-head form of the above ([batch, heads, seq, d],
 * caller's stream).  precision FA_NAIVE_F64 computes scores, softmax and PV
 * in f64 (output rounded to f32): an on-device reference for checking the
 * flash kernels at sizes a CPU oracle cannot reach.  The score buffer is
 * allocated stream-ordered for as many whole heads at a time as fit in both
 * 8 GiB and half the device memory free at the call (at least one head); a
 * single head's score matrix larger than half the free memory returns
 * FA_ERR_ALLOC with nothing queued.  No counterpart beyond naive_attention
 * itself in the reference. */
#define FA_NAIVE_F32 0
#define FA_NAIVE_F64 1
int fa_naive_device(void* stream, const float* q, const float* k, const float* v, size_t batch,
                    size_t heads, size_t seq_len_q, size_t seq_len_k, size_t d_head, int causal,
                    int precision, float* out);

/* ---- introspection -------------------------------------------------------
 * fa_init loads the code object on the current device (done lazily by every
 * entry point).  fa_describe_launch writes the kernel name(s) and grid the
 * given call would launch, e.g. "fa_prefill_v2_d128_1 grid=512x1x1 block=512",
 * launching nothing and needing no device (it plans for the current
 * device's CU count, or 256 CUs when no device is visible); it returns the
 * argument / support status the launch would return. */
int fa_init(void);
int fa_describe_launch(int variant, size_t batch, size_t heads, size_t seq_len_q, size_t seq_len_k,
                       size_t d_head, int causal, const fa_launch_opts* opts, char* buf,
                       size_t buf_len);

/* ---- peak probes ---------------------------------------------------------
 * No counterpart in the reference: a measurement aid, so the roofline
 * denominators (the MI355X data-sheet peaks) can be checked against the
 * machine.  Queues one probe kernel on `stream` (device memory `buf`, 16-byte
 * aligned, `bytes` long) and stores its work in *work; the caller times it.
 *   FA_PROBE_MFMA_*: every wave of 8 x #CUs four-wave workgroups (two
 *     resident per CU) runs independent chains of `iters` (1 .. 2^20)
 *     back-to-back MFMAs of that kind and writes one checksum float to buf
 *     (bytes >= 128 x #CUs); *work = FLOP.
 *   FA_PROBE_COPY: copies the first bytes/2 of buf (whole 16-byte elements)
 *     onto the second half;
 *   FA_PROBE_READ: reads the first bytes/2 of buf (whole 16-byte elements),
 *     each workgroup one contiguous chunk, and writes nothing; *work = bytes
 *     read;
 *     *work = bytes read + bytes written. */
#define FA_PROBE_MFMA_F32_32X32X2 0
#define FA_PROBE_MFMA_F32_16X16X4 1
#define FA_PROBE_MFMA_BF16_16X16X32 2
#define FA_PROBE_COPY 3
#define FA_PROBE_MFMA_BF16_32X32X16 4
#define FA_PROBE_READ 5
int fa_probe_launch(int kind, void* stream, void* buf, size_t bytes, unsigned iters, double* work);

#ifdef __cplusplus
}
#endif
#endif /* FA_HIP_H */
