// fa_kernels.hip -- gfx950 (CDNA4) kernels for the FlashAttention forward pass.
//
// Replaces the reference crate's per-variant tiling loops and Kernel-trait
// micro-kernels (amaye15/flash-attention-cpu):
//   run_v1  src/v1.rs:162-396   -> prefill_body<D, 1, LOADER>
//   run_v2  src/v2.rs:160-385   -> prefill_body<D, 2, LOADER>
//   run_v3  src/v3.rs:351-512   -> prefill_body<D, 3, LOADER>
//   dot4x4 / dot4 / dot         -> QK^T on v_mfma_f32_16x16x4_f32
//   max_reduce4 / sub_exp_sum4  -> per-lane max/exp2/sum + permlane swaps
//   pv4 / axpy / scale_inplace  -> PV on v_mfma_f32_16x16x4_f32, per-lane rescale
//   naive_attention src/naive.rs:14-75 -> naive_{scores,softmax,pv}_body
//   (new) split-KV + LSE merge  -> decode_body / merge_body (short queries,
//                                  and the prefill key split on small grids)
//
// All arithmetic is IEEE f32 (f32 MFMA, no reduced-precision inputs); the
// naive kernels also have an f64 instantiation for on-device checking.
//
// Prefill geometry (D = d_head padded to 32/64/128/256/512/1024; fa_params.h):
//   * a workgroup of NW = 8 waves owns BQ = 128 query rows of one
//     (batch*head) slice; wave w owns rows 16w .. 16w+15 (D > 256: column
//     groups of D/256 waves share a 16-row tile, 256 columns each);
//   * keys stream through LDS in stages of SK keys (64 for D <= 128, 32 or
//     16 for D = 256), K rows padded to D+8 floats and V rows to D+16 (D+8
//     at D = 32) so 128-bit reads are free of bank conflicts on the 128-bank
//     LDS; v3 double-buffers K and V and fills them by global->LDS DMA;
//   * scores are computed transposed, S^T = K Q^T (A = 16 K rows from LDS,
//     B = the wave's 16 Q rows held in VGPRs), so lane l owns query row l%16
//     and keys 4(l/16)+r of every 16-key block;
//   * the exp'd scores are then already the B operand of O^T = V^T P^T, and
//     each lane's O^T accumulators belong to its own query row, so the
//     online-softmax rescale is a per-lane multiply.
//
// MFMA operand layouts (verified on MI355X):
//   32x32x2 f32: A[i][k] in lane (i + 32k), B[k][j] in lane (j + 32k),
//                C[i][j] in lane (j + 32*((i/4)%2)), reg 4*(i/8) + i%4.
//   16x16x4 f32: A[i][k] in lane (i + 16k), B[k][j] in lane (j + 16k),
//                C[i][j] in lane (j + 16*(i/4)), reg i%4.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fa_params.h"

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define FA_NEG_INF (-__builtin_huge_valf())

// Prefill's lazy running max (log2 units): exponentials are taken against a
// reference that may trail the true row max by up to this much.
constexpr float kLazyMax = 8.0f;

#ifndef FA_DECODE_INTERLEAVE
#define FA_DECODE_INTERLEAVE 1
#endif
// Cache policy of the decode K DMA (buffer aux bits): 2 = nt, the stream is
// read once (measured on config 4b: 168.1 -> 162.8 us against 0).
#ifndef FA_DECODE_KLDS_AUX
#define FA_DECODE_KLDS_AUX 2
#endif
// v3 prefill: only the upper half of the waves issue the stage DMA.
#ifndef FA_FILL_HALF
#define FA_FILL_HALF 1
#endif
// v3 prefill, D = 128: the non-filling waves take each stage's softmax
// before the step's barrier, their partners after it.
#ifndef FA_SPLIT_SOFTMAX
#define FA_SPLIT_SOFTMAX 1
#endif

// ---------------------------------------------------------------------------
// Small device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float fa_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// exp(a - b) in the log2 domain for running maxima that may still be -inf
// (a row that has not seen a visible key yet): returns 0 when a == -inf.
__device__ __forceinline__ float rescale_factor(float m_old, float m_new, float c) {
    return (m_old == FA_NEG_INF) ? 0.0f : fa_exp2((m_old - m_new) * c);
}

// Four floats of row `row` from column `col` (zero outside [0,nrows) x [0,d)).
// NT: non-temporal load, for data streamed exactly once (split-KV K/V).
template <bool VEC, bool NT = false>
__device__ __forceinline__ f32x4 load4(const float* __restrict__ base, int row, int nrows, int col, int d) {
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (row < nrows) {
        const float* p = base + (size_t)row * d + col;
        if (VEC) {
            if (col < d) {
                if constexpr (NT) v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
                else v = *reinterpret_cast<const f32x4*>(p);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < d) v[e] = p[e];
        }
    }
    return v;
}

// Decode operand registers: f32x4 for f32 inputs; for 16-bit inputs the raw
// 4 elements, widened to f32 (exactly) only where the MFMA consumes them, so
// a prefetch does not wait for its load.
template <typename E>
struct RawOf {
    typedef E type __attribute__((ext_vector_type(4)));
};
template <>
struct RawOf<float> {
    typedef f32x4 type;
};
template <typename E>
__device__ __forceinline__ f32x4 widen(const typename RawOf<E>::type& r) {
    if constexpr (std::is_same<E, float>::value) {
        return r;
    } else {
        return (f32x4){static_cast<float>(r[0]), static_cast<float>(r[1]), static_cast<float>(r[2]),
                       static_cast<float>(r[3])};
    }
}
// load4 for any element type, raw (zero outside [0,nrows) x [0,d)).  VEC:
// one 16-byte (f32) or 8-byte (16-bit) load; d % 4 == 0 and aligned rows.
template <typename E, bool VEC, bool NT = false>
__device__ __forceinline__ typename RawOf<E>::type load4r(const E* __restrict__ base, int row, int nrows, int col,
                                                           int d) {
    typedef typename RawOf<E>::type R;
    if constexpr (std::is_same<E, float>::value) {
        return load4<VEC, NT>(base, row, nrows, col, d);
    } else {
        R v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = E(0.0f);
        if (row < nrows) {
            const E* p = base + (size_t)row * d + col;
            if (VEC) {
                if (col < d) {
                    unsigned long long bits;
                    if constexpr (NT) bits = __builtin_nontemporal_load(reinterpret_cast<const unsigned long long*>(p));
                    else bits = *reinterpret_cast<const unsigned long long*>(p);
                    v = __builtin_bit_cast(R, bits);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col + e < d) v[e] = p[e];
            }
        }
        return v;
    }
}

// Workgroup -> (query block, batch*head) with the longest causal blocks first
// (greedy longest-processing-time order as workgroups retire) and, when bh is
// a multiple of 8, all blocks of one head on the same XCD (workgroups are
// dispatched round-robin over the 8 XCDs) so its K/V stays in one L2.
__device__ __forceinline__ void map_block(const FaParams& p, int x, int& qb, int& bh) {
    int rank;
    if (p.bh % 8 == 0) {
        const int hpx = p.bh / 8;
        const int xcd = x % 8, s = x / 8;
        bh = (s % hpx) * 8 + xcd;
        rank = s / hpx;
    } else {
        bh = x % p.bh;
        rank = x / p.bh;
    }
    if (p.pair_w > 0) {
        // With two resident workgroups per CU, workgroups x and x + #CUs share
        // a CU; reversing every second round of ranks pairs the k-th longest
        // causal block with the k-th shortest.
        const int round = rank / p.pair_w, w_eff = min(p.pair_w, p.nqb - round * p.pair_w);
        if (round & 1) rank = round * p.pair_w + (w_eff - 1 - rank % p.pair_w);
    }
    qb = p.causal ? (p.nqb - 1 - rank) : rank;
}

// Two-block grid (bh * nqb / 2 workgroups, nqb even): workgroup x takes
// query blocks nqb-1-r and r of one (batch, head), with the (bh, r) order of
// map_block over nqb / 2 ranks.  Causal blocks r and nqb-1-r together cover
// nqb + 1 stage pairs, the same for every workgroup.
__device__ __forceinline__ void map_pair(const FaParams& p, int x, int& qa, int& qb2, int& bh) {
    int rank;
    if (p.bh % 8 == 0) {
        const int hpx = p.bh / 8;
        const int xcd = x % 8, s = x / 8;
        bh = (s % hpx) * 8 + xcd;
        rank = s / hpx;
    } else {
        bh = x % p.bh;
        rank = x / p.bh;
    }
    qa = p.nqb - 1 - rank;
    qb2 = rank;
}

// Key-split grid: a compact 1-D list of the workgroups that have keys to
// process (a grid padded with idle workgroups lets the dispatcher queue
// working ones behind busy CUs).  Row y holds split y of every query block
// whose key range reaches y * split_len -- causal blocks qb >= floor(y *
// split_len / ks_rows), all blocks otherwise (and for v1, whose blocks all
// visit every key) -- in map_block's order.
__device__ __forceinline__ void map_block_split(const FaParams& p, int& qb, int& bh, int& y) {
    int t = blockIdx.x;
    int cnt = p.nqb;
    for (y = 0;; ++y) {
        cnt = (p.causal && !p.full_keys) ? p.nqb - (int)(((long long)y * p.split_len) / p.ks_rows) : p.nqb;
        if (t < cnt * p.bh || y + 1 >= p.num_splits) break;
        t -= cnt * p.bh;
    }
    // rank r of this row is block nqb-1-r (causal) or r, as in map_block
    map_block(p, t, qb, bh);
}

// ---------------------------------------------------------------------------
// Prefill kernel: one template for v1 / v2 / v3.
//
// A workgroup of NW waves owns BQ = 16*NW query rows of one (batch*head)
// slice; wave w owns rows 16w .. 16w+15.  Keys stream through LDS in stages
// of SK keys shared by the workgroup's waves (fa_params.h: fa_prefill_*).
//
// Scores are computed transposed on 16x16x4 f32 MFMA, S^T = K Q^T: A = 16 K
// rows from LDS, B = the wave's 16 Q rows held in VGPRs.  Lane l then owns
// query row l%16 and keys 4*(l/16)+r (r = 0..3) of every 16-key block, so a
// row's max / sum spans the 4 lanes l%16 + 16k (two swaps).  The exp'd
// scores are already the B operand of O^T = V^T P^T, and lane l's O^T
// accumulators all belong to its own query row, so the online-softmax
// rescale is a per-lane multiply.  V is read with one 128-bit LDS read per
// 64 output columns: lane l reads V[key][64hh + 4(l%16) .. +3], so O^T block
// (hh, j) row i holds dv = 64hh + 4i + j.
//
// LDS holds K and V stages as padded rows: K rows of D + 8 floats, so the 32
// lanes a 128-bit read serves per cycle (16 rows x 2 adjacent chunks) hit 32
// distinct 4-bank groups of the 128 banks; V rows of D + 16 floats (D + 8
// for D = 32), so the 4 rows read together (4 lane groups x 16 contiguous
// chunks) sit 256 B apart modulo the bank width.  Every read address is a
// per-lane base plus an immediate offset.  The gfx950 global->LDS DMA writes
// 1 KB runs of this padded image; pad slots re-load a valid chunk.
//
// LOADER: 0 = scalar global loads through VGPRs (any d), 1 = 128-bit loads
// through VGPRs (d % 4 == 0), 2 = global_load_lds_dwordx4 DMA (d % 4 == 0,
// 16-byte aligned operands; v3 only).
// ---------------------------------------------------------------------------
// Padded LDS row lengths (floats) of the K and V stage images.
template <int D> constexpr int kpad_row() { return D + 8; }
template <int D> constexpr int vpad_row() { return D == 32 ? D + 8 : D + 16; }

template <int LD>
__device__ __forceinline__ int lds_off(int row, int chunk) {
    return row * LD + 4 * chunk;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    // s_waitcnt with vmcnt = N and expcnt / lgkmcnt left at their maxima.
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// max / sum over the 4 lanes (l%16 + 16k) that hold one query row.  Both
// swaps hand every lane the pair in the same order, so all 4 lanes end
// with bit-identical results.
// max(a, b) as med3(a, b, +inf): one v_med3_f32, where fmaxf on values the
// compiler cannot prove canonical (cross-lane moves, MFMA results) costs two
// extra canonicalising v_max_f32.  The empty asm hides the constant so the
// compiler cannot turn the med3 back into that max.  Differs from fmaxf
// only for NaN inputs.
__device__ __forceinline__ float fmax_fast(float a, float b) {
    float inf = __builtin_huge_valf();
    asm("" : "+s"(inf));
    return __builtin_amdgcn_fmed3f(a, b, inf);
}
__device__ __forceinline__ float row4_max(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmax_fast(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmax_fast(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row4_sum(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 4 x 4 transpose over (16-lane group g, register r) of four f32x4 values:
// afterwards v[r] of lane group g holds what v[g] of lane group r held.  Two
// permlane-swap levels (halves, then 16-lane rows), as in row4_max.  Used to
// turn an O^T tile's "columns 64 hh + 4 (4 g + r)" into "columns 64 hh + 16 r
// + 4 g", so a store instruction writes 64 contiguous bytes of every row.
__device__ __forceinline__ void lane_group_transpose4(float (&v)[4][4]) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[r][e]), __float_as_uint(v[r + 2][e]),
                                                            false, false);
            v[r][e] = __uint_as_float(t[0]);
            v[r + 2][e] = __uint_as_float(t[1]);
        }
#pragma unroll
    for (int r = 0; r < 4; r += 2)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[r][e]), __float_as_uint(v[r + 1][e]),
                                                            false, false);
            v[r][e] = __uint_as_float(t[0]);
            v[r + 1][e] = __uint_as_float(t[1]);
        }
}

// One workgroup's share of a query block: query block qb of slice bh (and,
// in the two-block grid, block qb_second after it), key stages sbeg ..
// sbeg + nst - 1 of the block's range (nst < 0: to its end); slot >= 0
// writes a partial (m, l, O) into split slot `slot` for fa_merge, slot < 0
// the normalised rows.
struct PrefillSeg {
    int qb, bh, qb_second, sbeg, nst, slot;
};

template <int D, int VARIANT, int LOADER, bool STREAM, bool OPAQUE_TID>
__device__ __forceinline__ void prefill_segment(const FaParams& p, const PrefillSeg& seg) {
    constexpr int NW = fa_prefill_waves(D);   // waves per workgroup
    constexpr int NT = NW * 64;               // threads
    constexpr int BQ = fa_prefill_rows(D);    // query rows per workgroup
    constexpr int SK = fa_prefill_stage_keys(D, VARIANT);   // keys per LDS stage
    constexpr int KB = SK / 16;               // 16-key blocks per stage
    // Column groups (D > 256): CG waves share a 16-row tile, each holding DW
    // columns of Q and O; their partial scores are summed through LDS.
    constexpr int CG = fa_prefill_cgroups(D);
    constexpr int DW = D / CG;                // columns per wave
    constexpr int TILES = NW / CG;            // 16-row tiles per workgroup
    constexpr int NQ = DW / 4;                // MFMA k-steps over the wave's columns
    constexpr int NC = DW / 16;               // 128-bit K reads per lane per key block
    constexpr int VW = (DW >= 64) ? 4 : 2;    // floats per lane per V read
    constexpr int NVR = (DW >= 64) ? DW / 64 : 1;   // V reads per key
    constexpr int NOB = DW / 16;              // O^T accumulator blocks
    constexpr int CPR = D / 4;                // 16-byte chunks per row
    constexpr int LDK = kpad_row<D>();        // padded K row (floats)
    constexpr int LDV = vpad_row<D>();        // padded V row (floats)
    constexpr int KTILE = SK * LDK;           // floats per K stage
    constexpr int VTILE = SK * LDV;           // floats per V stage
    constexpr bool DMA = (LOADER == 2);
    constexpr int NBUF = fa_prefill_nbuf(D, VARIANT);
    constexpr bool PIPE = NBUF == 2;          // v3's double-buffered schedule
    // v3 where one K + V stage is all the LDS holds (D = 1024): the K and V
    // buffers alternate (V of a stage streams in under its QK^T, K of the
    // next under its softmax + PV)
    constexpr bool KVPP = VARIANT == 3 && !PIPE && DMA;
    static_assert(NVR * VW == NOB, "V read layout");
    static_assert(!DMA || PIPE || KVPP, "LDS DMA needs one of v3's overlapped schedules");
    static_assert((SK * CPR) % NT == 0, "stage load must split evenly");
    static_assert(BQ == 16 * TILES && CG * DW == D, "column groups");

    // D = 2048: one 16-key stage of K or V takes 129 KiB, so K and V take
    // turns in one buffer (Kb0, sized for the longer V rows).
    constexpr bool KV1 = D > 1024;
    static_assert(!KV1 || (!PIPE && !DMA), "the shared K / V buffer is register-filled, one stage");
    // Separate arrays so the compiler can tell a DMA in flight into one
    // buffer from LDS reads of another (no needless vmcnt waits).
    __shared__ __attribute__((aligned(16))) float Kb0[KV1 ? (KTILE > VTILE ? KTILE : VTILE) : KTILE];
    __shared__ __attribute__((aligned(16))) float Vb0[KV1 ? 4 : VTILE];
    __shared__ __attribute__((aligned(16))) float Kb1[NBUF > 1 ? KTILE : 4];
    __shared__ __attribute__((aligned(16))) float Vb1[NBUF > 1 ? VTILE : 4];
    // Column groups: per-wave partial scores, one slot per wave (two in the
    // pipelined schedule, which has one barrier per stage).
    constexpr int XSLOTS = CG > 1 ? (PIPE ? 2 : 1) : 0;
    __shared__ __attribute__((aligned(16))) f32x4 Xs[XSLOTS ? XSLOTS * NW * KB * 64 : 1];

    int tid = threadIdx.x;
    // In the stream split's segment loop, an opaque tid keeps per-lane
    // addresses from being hoisted out of the loop and held in VGPRs across
    // every stage loop.
    if constexpr (OPAQUE_TID) asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = CG > 1 ? wave % TILES : wave;   // the wave's 16-row tile
    const int cgrp = CG > 1 ? wave / TILES : 0;      // its column group
    const int c0 = cgrp * DW;                 // its first column of Q and O
    const int g = lane >> 4;                  // lane group 0..3
    const int li = lane & 15;

    // Split kernels (STREAM): this segment writes a partial -- a piece of a
    // stream-split block shared with other workgroups, or a key split
    const bool splitk = STREAM && seg.slot >= 0;
    // two_blocks (v3, no key split): this workgroup runs query blocks
    // nqb-1-r and then r of one (batch, head) -- equal causal work per
    // workgroup, and the second block's loads overlap the first's last step.
    const bool pairs = !STREAM && VARIANT == 3 && D == 128 && !splitk && p.two_blocks != 0;
    const int qb = seg.qb, bh = seg.bh, ysplit = seg.slot, qb_second = seg.qb_second;
    const int seq_q = p.seq_q, seq_k = p.seq_k, d = p.d;
    int q0 = qb * BQ;
    const float* __restrict__ Qh = p.q + (size_t)bh * seq_q * d;
    const float* __restrict__ Kh = p.k + (size_t)bh * seq_k * d;
    const float* __restrict__ Vh = p.v + (size_t)bh * seq_k * d;
    float* __restrict__ Oh = p.out + (size_t)bh * seq_q * d;
    const float c = p.scale_log2e;
    const bool causal = p.causal != 0;

    // Q rows of this wave as the B operand: lane holds Q[row][c0 + 16cc + 4g
    // + i], pre-multiplied by scale * log2(e) so scores come out of the MFMA
    // in the exp2 domain (src/v2.rs:171-173 multiplies after the dot; the
    // product differs by one f32 rounding per element of Q).
    int row_first = q0 + 16 * tile;
    int qrow = row_first + li;
    float qreg[NQ];
    auto load_q = [&](int row) {   // unscaled
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
            const f32x4 t = load4<LOADER != 0>(Qh, row, seq_q, c0 + 16 * cc + 4 * g, d);
#pragma unroll
            for (int i = 0; i < 4; ++i) qreg[4 * cc + i] = t[i];
        }
    };
    auto scale_q = [&]() {
#pragma unroll
        for (int i = 0; i < NQ; ++i) qreg[i] *= c;
    };
    // LATE_Q (v3 with the DMA loader, D = 128 and 256, split kernels too): Q
    // is loaded after the first stages' DMA is issued and scaled chunk by
    // chunk inside stage 0's QK^T, so the first MFMAs wait for K(0) and Q's
    // first chunk only (below).  Measured on MI355X, bit-identical outputs:
    // config 3 3976 -> 3962 us, config 5's shape 546.7 -> 542.8 us, config 2
    // and config 5c unchanged.
    constexpr bool LATE_Q = PIPE && DMA && CG == 1 && (D == 128 || D == 256);
    if constexpr (!LATE_Q) {
        load_q(qrow);
        scale_q();
    }

    f32x4 o[NOB];
#pragma unroll
    for (int j = 0; j < NOB; ++j) o[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    float m = FA_NEG_INF;   // reference max of the row's log2-domain scores (same in its 4 lanes)
    float l = 0.0f;         // v2/v3: this lane's partial row sum; v1: full row sum
    // v1: whether the current stage changes the row (some probability above
    // zero, or a rescale); a stage that does not -- keys past the row's
    // causal end, which v1 still visits -- skips the un-normalise /
    // re-normalise round trip, an identity whose two roundings (o * l, then
    // o * fl(1/l)) would otherwise drift o once per such stage.
    bool v1_moves = true;
    // -m (0 while m = -inf) as the QK^T chain's initial accumulator: the MFMA
    // then yields S - m directly, with no per-score subtraction.
    f32x4 nref = {0.0f, 0.0f, 0.0f, 0.0f};

    // Keys this workgroup visits: v1 visits every key (no causal skip,
    // src/v1.rs:209-216); v2/v3 stop after the block's last diagonal key
    // (src/v2.rs:208-212, src/v3.rs:396-410).
    auto block_end = [&](int q0_) { return (VARIANT != 1 && causal) ? min(seq_k, q0_ + BQ) : seq_k; };
    int kend = block_end(q0);
    // Key split / stream split (v2/v3 on grids smaller than the GPU): this
    // workgroup takes stages sbeg .. sbeg + nst - 1 of the block's range
    // (sbeg < the block's stage count by construction of the grid).
    const int sbeg = seg.sbeg;
    int nst = (kend + SK - 1) / SK - sbeg;
    if (seg.nst >= 0) nst = min(nst, seg.nst);
    const int k0 = sbeg * SK;                 // first key of this workgroup

    // ---- stage loaders ------------------------------------------------------
    constexpr int LOAD_ITERS = (SK * CPR) / NT;
    auto load_regs = [&](const float* __restrict__ src, int kbase, f32x4* rg) {
#pragma unroll
        for (int it = 0; it < LOAD_ITERS; ++it) {
            const int idx = tid + it * NT;
            rg[it] = load4<LOADER != 0>(src, kbase + idx / CPR, seq_k, 4 * (idx % CPR), d);
        }
    };
    auto store_regs = [&](auto ld, float* dst, const f32x4* rg) {
        constexpr int LD = decltype(ld)::value;
#pragma unroll
        for (int it = 0; it < LOAD_ITERS; ++it) {
            const int idx = tid + it * NT;
            *reinterpret_cast<f32x4*>(dst + lds_off<LD>(idx / CPR, idx % CPR)) = rg[it];
        }
    };
    // DMA: the stage image is SK rows of LD/4 chunks (the last ones are the
    // pad); run R = i*FW + f (64 chunks = 1 KB) is written by filling wave f,
    // lane L fetching the global chunk that belongs at image position 64R + L
    // (columns past d and pad slots fetch column 0).  Every stage is fetched
    // with buffer loads: a per-stage buffer resource (base = the stage's
    // first row, range ending at seq_k, in SGPRs) and per-lane byte offsets
    // that are the same for every stage, computed once below -- no per-stage
    // VALU address arithmetic.
    // Only the FW highest-numbered waves fill (all NW without the DMA
    // loader).  Waves w and w + NW/2 share a SIMD and the lower-numbered one
    // wins MFMA issue, so v3 leaves the stage's DMA to waves NW/2 .. NW-1:
    // after each barrier their partners go straight to softmax and MFMA work
    // while the fill instructions queue on the CU's load path.  Measured per
    // wave (s_memtime): with every wave filling, each spent 0.9-1.3k cycles
    // per stage issuing its DMA right after the barrier, with neither wave of
    // a SIMD issuing MFMAs meanwhile.
    constexpr int FW = (DMA && FA_FILL_HALF && PIPE) ? NW / 2 : NW;
    const int fwave = wave - (NW - FW);   // index among the filling waves; < 0: does not fill
    auto dma_geometry = [&](auto ld, int* voff) {
        constexpr int RCH = decltype(ld)::value / 4;   // chunks per padded row
        constexpr int TOTAL = SK * RCH;
        constexpr int RUNS = (TOTAL + 63) / 64;
        constexpr int NI = (RUNS + FW - 1) / FW;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int pos = (i * FW + fwave) * 64 + lane;
            const int r = pos / RCH, cidx = pos % RCH;
            const int col = (cidx < CPR && 4 * cidx < d) ? 4 * cidx : 0;
            voff[i] = (fwave >= 0 && pos < TOTAL) ? 4 * (r * d + col) : -1;   // -1: lane past the image
        }
    };
    auto dma_stage = [&](auto ld, const float* __restrict__ src, int kbase, float* dst, const int* voff) {
        constexpr int RCH = decltype(ld)::value / 4;
        constexpr int TOTAL = SK * RCH;
        constexpr int RUNS = (TOTAL + 63) / 64;
        constexpr int NI = (RUNS + FW - 1) / FW;
        if (fwave < 0) return;
        // The resource's range ends at seq_k: in the last, partial stage the
        // rows past it read as zeros (measured on MI355X: out-of-range lanes
        // of an LDS-DMA buffer load write 0 to LDS), and their scores are
        // masked to -inf, so full and partial stages share one path.
        const int rows = min(SK, seq_k - kbase);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(src + (size_t)kbase * d), (short)0, rows * d * 4, 0x00020000);
        // LDS destinations from one opaque per-stage base: the compiler
        // would otherwise keep every run's address in its own SGPR.
        int w256 = fwave * 256;
        asm volatile("" : "+s"(w256));
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int run = i * FW + fwave;
            // every filling wave has run i < RUNS while (i + 1) * FW <= RUNS;
            // only the image's last run can have lanes past it
            if (((i + 1) * FW <= RUNS || run < RUNS) && (TOTAL % 64 == 0 || run < RUNS - 1 || voff[i] >= 0))
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs, (__attribute__((address_space(3))) void*)(dst + i * FW * 256 + w256), 16, voff[i], 0, 0, 0);
        }
    };
    constexpr int NI_K = ((SK * (LDK / 4) + 63) / 64 + FW - 1) / FW;
    constexpr int NI_V = ((SK * (LDV / 4) + 63) / 64 + FW - 1) / FW;
    int voff_k[DMA ? NI_K : 1], voff_v[DMA ? NI_V : 1];
    if constexpr (DMA) {
        dma_geometry(std::integral_constant<int, LDK>{}, voff_k);
        dma_geometry(std::integral_constant<int, LDV>{}, voff_v);
    }
    auto fill_stage = [&](auto ld, const float* __restrict__ src, int kbase, float* dst) {
        if constexpr (DMA) {
            dma_stage(ld, src, kbase, dst, decltype(ld)::value == LDK ? voff_k : voff_v);
        } else {
            f32x4 rg[LOAD_ITERS];
            load_regs(src, kbase, rg);
            store_regs(ld, dst, rg);
        }
    };
    const std::integral_constant<int, LDK> KL{};
    const std::integral_constant<int, LDV> VL{};

    // ---- stage math ---------------------------------------------------------
    // S^T - m for the stage's KB key blocks from `Ks` (each chain starts from
    // nref = -m).  An MFMA chain rounds like a sequential FMA loop, and f32
    // VALU work does not overlap f32 MFMA on gfx950 (an f32 MFMA holds the
    // SIMD's VALU issue for its 32 cycles), so the summation order trades
    // accuracy against VALU adds:
    //  * D <= 128: one chain over d per key block (N(0,1)-scale logits keep
    //    its rounding far inside the f32 parity bar);
    //  * D = 256: each 128-bit K read feeds a fresh 4-step (16-product) chain
    //    that is added to the running sum -- blocks of 16 bring the error down
    //    to that of the crate's 16-lane AVX-512 dot products
    //    (src/avx512.rs:195-234), which config 5's large logits need.
    constexpr bool BLOCKED_QK = D > 128;
    // Read-ahead: the first PRE d-chunks of the next QK^T and the first PRE
    // V steps of the next PV are read into registers before the softmax VALU
    // work (the stage is already resident), so their LDS latency is hidden;
    // inside QK^T and PV the reads then run PRE chunks / steps ahead through
    // a ring of PRE + 1 register sets, each read issued after the MFMAs that
    // last used its slot.  D = 256: v2 runs one ahead (230 VGPRs; config 5's
    // shape 577 -> 572.5 us); v1 gains nothing and v3, with its second K / V
    // buffer, would spill, so they read each operand just before its MFMA
    // (as does v2 at D = 1024, where the scalar loader would spill).
    constexpr int PRE = (DW <= 128) ? 2 : (VARIANT == 2 && D <= 512 ? 1 : 0);
    f32x4 kpre[PRE ? PRE : 1][KB];
    auto k_chunk = [&](const float* Ks, int cc, f32x4* dst) {
#pragma unroll
        for (int b = 0; b < KB; ++b)
            dst[b] = *reinterpret_cast<const f32x4*>(Ks + lds_off<LDK>(16 * b + li, c0 / 4 + 4 * cc + g));
    };
    auto qk_preload = [&](const float* Ks) {
        if constexpr (PRE > 0) {
#pragma unroll
            for (int cc = 0; cc < PRE && cc < NC; ++cc) k_chunk(Ks, cc, kpre[cc]);
        }
    };
    auto qk_mfma = [&](const f32x4* kk, int cc, f32x4* s) {
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            if constexpr (BLOCKED_QK) {
                f32x4 t = (cc == 0) ? nref : (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    t = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[b][i], qreg[4 * cc + i], t, 0, 0, 0);
                s[b] = (cc == 0) ? t : s[b] + t;
            } else {
                f32x4& acc = s[b];
                if (cc == 0) acc = nref;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[b][i], qreg[4 * cc + i], acc, 0, 0, 0);
            }
        }
    };
    // SCALE: multiply each Q chunk by scale * log2(e) right before its
    // MFMAs (stage 0 of LATE_Q, where Q arrives chunk by chunk); the factor
    // passes through an empty asm there so the multiplies, and the waits for
    // their loads, stay with their own chunk.
    auto qk_stage = [&](const float* Ks, f32x4* s, auto scale_c) {   // after qk_preload(Ks)
        constexpr bool SCALE = decltype(scale_c)::value;
        auto scale_chunk = [&](int cc) {
            if constexpr (SCALE) {
                float cs = c;
                asm volatile("" : "+s"(cs));
#pragma unroll
                for (int i = 0; i < 4; ++i) qreg[4 * cc + i] *= cs;
            }
        };
        if constexpr (PRE > 0) {
            constexpr int KR = PRE + 1;
            f32x4 kk[KR][KB];
#pragma unroll
            for (int cc = 0; cc < PRE && cc < NC; ++cc)
#pragma unroll
                for (int b = 0; b < KB; ++b) kk[cc][b] = kpre[cc][b];
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) {
                scale_chunk(cc);
                qk_mfma(kk[cc % KR], cc, s);
                if (cc + PRE < NC) k_chunk(Ks, cc + PRE, kk[(cc + PRE) % KR]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            // K operands one chunk ahead; a scheduling barrier per chunk keeps
            // the live set to two chunks' reads.
            f32x4 kk[2][KB];
            k_chunk(Ks, 0, kk[0]);
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) {
                if (cc + 1 < NC) k_chunk(Ks, cc + 1, kk[(cc + 1) & 1]);
                scale_chunk(cc);
                qk_mfma(kk[cc & 1], cc, s);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // Mask keys >= seq_k and, when causal, keys > query row (top-left
    // aligned, src/naive.rs:37; diagonal stages only, src/v2.rs:268-287).
    auto mask_stage = [&](f32x4* s, int kbase) {
        const bool need = (kbase + SK > seq_k) || (causal && kbase + SK - 1 > row_first);
        if (need) {
#pragma unroll
            for (int b = 0; b < KB; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = kbase + 16 * b + 4 * g + r;
                    if (key >= seq_k || (causal && key > qrow)) s[b][r] = FA_NEG_INF;
                }
        }
    };

    // Column groups: each wave's QK^T covers its DW columns (group 0's chain
    // starts from -m); xs_put stores that partial in the wave's slot and,
    // after a barrier, xs_sum adds the tile's CG partials in group order, so
    // every wave of the tile holds bit-identical scores and runs the same
    // softmax (m, l and the lazy-max decisions agree across the group).
    auto xs_put = [&](const f32x4* s, int slot) {
        if constexpr (CG > 1) {
#pragma unroll
            for (int b = 0; b < KB; ++b) Xs[((slot * NW + wave) * KB + b) * 64 + lane] = s[b];
        }
    };
    auto xs_sum = [&](f32x4* s, int slot) {
        if constexpr (CG > 1) {
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                f32x4 t = Xs[((slot * NW + tile) * KB + b) * 64 + lane];
#pragma unroll
                for (int j = 1; j < CG; ++j) t += Xs[((slot * NW + j * TILES + tile) * KB + b) * 64 + lane];
                s[b] = t;
            }
        }
    };

    // V operands of PV step `step` (keys 16(step/4) + 4g + step%4).
    auto read_v = [&](const float* Vs, int step, f32x4* vv) {
        const int kr = 16 * (step / 4) + 4 * g + (step % 4);
#pragma unroll
        for (int hh = 0; hh < NVR; ++hh) {
            if constexpr (VW == 4) {
                vv[hh] = *reinterpret_cast<const f32x4*>(Vs + lds_off<LDV>(kr, c0 / 4 + 16 * hh + li));
            } else {
                const f32x2 t = *reinterpret_cast<const f32x2*>(Vs + lds_off<LDV>(kr, li >> 1) + 2 * (li & 1));
                vv[hh] = (f32x4){t[0], t[1], 0.0f, 0.0f};
            }
        }
    };
    f32x4 vpre[PRE ? PRE : 1][NVR];
    auto pv_preload = [&](const float* Vs) {
        if constexpr (PRE > 0) {
#pragma unroll
            for (int st = 0; st < PRE; ++st) read_v(Vs, st, vpre[st]);
        }
    };

    // Online-softmax update + PV for one stage (src/v2.rs:289-372; v1's
    // normalise / un-normalise round trip, src/v1.rs:291-385).  After
    // pv_preload(Vs).
    // softmax_part: turns s into probabilities and updates m, l (rescaling
    // o); pv_part: O^T += V^T P^T from them.  pv_hook(step) runs after each
    // PV step's MFMAs and V read-ahead.
    auto softmax_part = [&](f32x4* s) {
        // s holds S - m (S itself while m = -inf: nref was 0).
        float mt = fmax_fast(s[0][0], s[0][1]);
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
            for (int r = (b == 0) ? 2 : 0; r < 4; ++r) mt = fmaxf(mt, s[b][r]);
        // Lazy reference max: it moves only when the stage max exceeds it by
        // more than kLazyMax (log2 units), so exponentials stay <= 2^kLazyMax
        // and rescaling the accumulators is rare; otherwise nothing changes.
        // The final O / l is the same quotient (each term and l share the
        // reference), to f32 rounding.  The row's maximum (a reduction over
        // its 4 lanes) is needed only when some lane's own maximum passes the
        // threshold.
        const bool seen = m != FA_NEG_INF;
        const float thr = seen ? kLazyMax : FA_NEG_INF;   // from m = -inf: any visible key
        bool grow = false;
        float delta = 0.0f;                                // the reference moves up by delta
        if (__builtin_amdgcn_ballot_w64(mt > thr) != 0) {
            mt = row4_max(mt);
            grow = mt > thr;
            delta = grow ? mt : 0.0f;
#pragma unroll
            for (int b = 0; b < KB; ++b) s[b] -= delta;
            if (grow) m = (seen ? m : 0.0f) + delta;
            const float nm = (m == FA_NEG_INF || cgrp != 0) ? 0.0f : -m;   // -m only in group 0's chain
            nref = (f32x4){nm, nm, nm, nm};
        }
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) s[b][r] = fa_exp2(s[b][r]);
        float ps = s[0][0];
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
            for (int r = (b == 0) ? 1 : 0; r < 4; ++r) ps += s[b][r];
        // A row seen before whose reference moved scales o and l by
        // 2^-delta; a row with none before has o = l = 0 (no factor needed).
        const bool rescale = grow && seen;
        if (VARIANT == 1) {
            const float corr = rescale ? fa_exp2(-delta) : 1.0f;
            const float rs = row4_sum(ps);
            const float l_new = corr * l + rs;
            v1_moves = rescale || rs != 0.0f;
            const float f = v1_moves ? l * corr : 1.0f;
#pragma unroll
            for (int j = 0; j < NOB; ++j) o[j] *= f;
            l = l_new;
        } else {
            // skipped unless some row of the wave rescales
            if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
                const float corr = rescale ? fa_exp2(-delta) : 1.0f;
                l *= corr;
#pragma unroll
                for (int j = 0; j < NOB; ++j) o[j] *= corr;
            }
            l += ps;
        }
    };
    auto pv_part = [&](const f32x4* s, const float* Vs, auto&& pv_hook) {
        // O^T += V^T P^T: 4 keys per MFMA step (key 16b + 4g + r in lane group
        // g), a scheduling barrier per step.
        auto pv_step = [&](int step, const f32x4* vv) {
            const float pr = s[step / 4][step % 4];
#pragma unroll
            for (int hh = 0; hh < NVR; ++hh)
#pragma unroll
                for (int j = 0; j < VW; ++j)
                    o[VW * hh + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[hh][j], pr, o[VW * hh + j], 0, 0, 0);
        };
        if constexpr (PRE > 0) {
            constexpr int VR = PRE + 1;
            f32x4 vv[VR][NVR];
#pragma unroll
            for (int st = 0; st < PRE; ++st)
#pragma unroll
                for (int hh = 0; hh < NVR; ++hh) vv[st][hh] = vpre[st][hh];
#pragma unroll
            for (int step = 0; step < 4 * KB; ++step) {
                pv_step(step, vv[step % VR]);
                if (step + PRE < 4 * KB) read_v(Vs, step + PRE, vv[(step + PRE) % VR]);
                pv_hook(step);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            f32x4 vv[NVR];   // d = 256: no read-ahead (registers)
#pragma unroll
            for (int step = 0; step < 4 * KB; ++step) {
                read_v(Vs, step, vv);
                pv_step(step, vv);
                pv_hook(step);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (VARIANT == 1) {
            const float inv = !v1_moves ? 1.0f : (l > 0.0f ? 1.0f / l : 0.0f);
#pragma unroll
            for (int j = 0; j < NOB; ++j) o[j] *= inv;
        }
    };
    auto no_hook = [](int) {};

    // Is this wave's share of stage `st` worth computing?  v2/v3 skip stages
    // entirely in the future of every row of the wave; v1 does not.
    auto stage_active = [&](int st) -> bool {
        const int kbase = k0 + st * SK;
        if (kbase >= seq_k) return false;
        if (VARIANT != 1 && causal && kbase > row_first + 15) return false;
        return true;
    };

    // Final normalisation with the l > 0 guard (src/v2.rs:375-382; v1's
    // accumulator is already normalised, src/v1.rs:389-393).
    // The O chunks this lane stores for column group hh, scaled by inv, in
    // row order (lane_group_transpose4): each store instruction then writes
    // 64 contiguous bytes of every row instead of 16-byte pieces 64 bytes
    // apart.
    auto row_chunks = [&](int hh, float inv, f32x4* x) {
        float v[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[r][e] = o[4 * hh + e][r] * inv;
        lane_group_transpose4(v);
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = (f32x4){v[r][0], v[r][1], v[r][2], v[r][3]};
    };
    // Row-order stores where measured faster (MI355X, bit-identical): config 5
    // v1 / v2 / v3 610.3 / 570.7 / 543.2 -> 602.3 / 559.7 / 536.4 us, config 2
    // v1 / v2 559.6 / 288.0 -> 557.5 / 285.7 us.  Not for the v3 D = 128
    // kernel (config 3 3965 -> 4001 us) nor the split kernels (config 5c
    // 0.2-1.0 us slower), which keep the register-order stores below.
    constexpr bool ROW_STORES = VW == 4 && !(VARIANT == 3 && D == 128) && !STREAM;
    auto write_out = [&]() {
        float inv = 1.0f;
        if (VARIANT != 1) {
            const float lt = row4_sum(l);
            inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        }
        if constexpr (ROW_STORES) {
            float* orow = Oh + (size_t)qrow * d;
#pragma unroll
            for (int hh = 0; hh < NVR; ++hh) {
                f32x4 x[4];
                row_chunks(hh, inv, x);   // every lane takes part in the swaps
                if (qrow < seq_q) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int dv0 = c0 + 64 * hh + 16 * k + 4 * g;
                        if (LOADER != 0 && dv0 + 4 <= d) {
                            *reinterpret_cast<f32x4*>(orow + dv0) = x[k];
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                if (dv0 + j < d) orow[dv0 + j] = x[k][j];
                        }
                    }
                }
            }
            return;
        }
        if (qrow < seq_q) {
            float* orow = Oh + (size_t)qrow * d;
#pragma unroll
            for (int hh = 0; hh < NVR; ++hh)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int dv0 = c0 + 64 * hh + VW * (4 * g + r);
                    if (LOADER != 0 && dv0 + VW <= d) {
                        if constexpr (VW == 4) {
                            const f32x4 t = {o[4 * hh][r] * inv, o[4 * hh + 1][r] * inv, o[4 * hh + 2][r] * inv,
                                             o[4 * hh + 3][r] * inv};
                            *reinterpret_cast<f32x4*>(orow + dv0) = t;
                        } else {
                            const f32x2 t = {o[0][r] * inv, o[1][r] * inv};
                            *reinterpret_cast<f32x2*>(orow + dv0) = t;
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < VW; ++j)
                            if (dv0 + j < d) orow[dv0 + j] = o[VW * hh + j][r] * inv;
                    }
                }
        }
    };

    if constexpr (PIPE) {
        // Double-buffered K and V (src/v3.rs:445-483: the next tile's scores
        // are issued before the current tile is finished).  At step st, K(st+2)
        // and V(st+1) stream by DMA into the buffers freed by the previous
        // step while this step computes from resident data; stage st+1's QK^T
        // is issued right after stage st's softmax + PV, and one barrier
        // closes the step.  The loop is unrolled by two so every buffer is a
        // compile-time choice.
        // With two blocks the stages of both run as one sequence g = 0 ..
        // nA + nB - 1 (block A: stages 0 .. nA-1), so the K/V loads of
        // block B's first stages are issued during block A's last steps like
        // any other; block B's Q is loaded at the start of A's last step (Q is
        // idle there) and the switch happens between that step's PV and the
        // QK^T of B's first stage.
        const int nA = nst;
        const int q0_b = qb_second * BQ;
        const int nB = pairs ? (block_end(q0_b) + SK - 1) / SK : 0;
        const int ntot = nA + nB;
        auto kb_of = [&](int gs) { return gs < nA ? k0 + gs * SK : (gs - nA) * SK; };
        auto gstage_active = [&](int gs) -> bool {
            const int kbase = kb_of(gs);
            const int rf = (gs < nA ? qb * BQ : q0_b) + 16 * tile;
            return kbase < seq_k && !(causal && kbase > rf + 15);
        };
        if constexpr (LATE_Q) {
            // The filling waves issue the DMA of K(0), V(0) and K(1), then
            // every wave its Q rows as NC buffer loads (with global loads in
            // flight next to the DMA the compiler ignores the explicit
            // vmcnt below and waits for every load before the first LDS read;
            // buffer loads it counts in order with the DMA).  VMEM loads of a
            // wave complete in order, so vmcnt(N), N = the fewest loads any
            // filling wave issues after K(0) (a partial last run still issues:
            // some of its lanes are in range), waits for K(0) alone; the bare
            // barrier (a workgroup fence would wait for every load) then
            // publishes it, and stage 0's QK^T waits for each Q chunk as it
            // uses it.
            constexpr int RUNS_K = (SK * (LDK / 4) + 63) / 64, RUNS_V = (SK * (LDV / 4) + 63) / 64;
            constexpr int AFTER_K0 = RUNS_V / FW + RUNS_K / FW + NC;
            // Issued whatever ntot is (with fewer than two stages the
            // spare fills repeat stage 0, in range and never read), so every
            // filling wave issues the same count on one path.
            const int kb0 = ntot > 0 ? kb_of(0) : 0, kb1 = ntot > 1 ? kb_of(1) : kb0;
            fill_stage(KL, Kh, kb0, Kb0);
            fill_stage(VL, Vh, kb0, Vb0);
            fill_stage(KL, Kh, kb1, Kb1);
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("" ::: "memory");
            {
                // rows past seq_q and columns past d read as 0 (out of range)
                const int rf = __builtin_amdgcn_readfirstlane(row_first);
                const int rows = __builtin_amdgcn_readfirstlane(max(0, min(16, seq_q - rf)));
                const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<float*>(Qh + (size_t)rf * d), (short)0, rows * d * 4, 0x00020000);
#pragma unroll
                for (int cc = 0; cc < NC; ++cc) {
                    const int col = c0 + 16 * cc + 4 * g;
                    const int off = col < d ? 4 * (li * d + col) : 0x7ffffff0;
                    const f32x4 t = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
#pragma unroll
                    for (int i = 0; i < 4; ++i) qreg[4 * cc + i] = t[i];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<AFTER_K0>();
            asm volatile("s_barrier" ::: "memory");
        } else {
            // Q and K(0) first; V(0) and K(1) stream in under stage 0's QK^T.
            if (ntot > 0) fill_stage(KL, Kh, kb_of(0), Kb0);
            wait_vmcnt<0>();
            __syncthreads();
            if (ntot > 0) fill_stage(VL, Vh, kb_of(0), Vb0);
            if (ntot > 1) fill_stage(KL, Kh, kb_of(1), Kb1);
        }
        // Waves w and w + NW/2 share a SIMD and the lower-numbered one wins
        // MFMA issue.  With the half fill, those (non-filling) waves take
        // each stage's softmax right after its QK^T, before the barrier that
        // ends the previous step -- while their partners still issue MFMAs --
        // and begin every step with PV MFMAs; their partners keep the
        // softmax at the start of the step, under the priority waves' MFMAs.
        // Same operations in the same order per wave; only the barrier moves.
        // Measured: d = 256 558.6 -> 548.9 us (config 5 shape), d = 64
        // 144.3 -> 143.2 us.  Not at D = 128, where the two loop copies
        // together need more than 256 VGPRs (39 spilled; 274 -> 288 us).
        constexpr bool EARLY_OK = D != 128 && CG == 1;
        const bool early = EARLY_OK && FW < NW && fwave < 0;
        // D = 128: the same split of the softmax between the two waves of a
        // SIMD within one loop copy -- the softmax has two call sites in the
        // step, taken by a wave-uniform flag (the barrier stays put; same
        // registers as one order).  Measured: config 2 272.1 -> 269.2 us,
        // config 3 4016 -> 3975 us, 32 x 2048^2 non-causal 513.6 -> 507.3 us.
        constexpr bool SPLIT_SM = FA_SPLIT_SOFTMAX && D == 128 && CG == 1;
        const bool sm_late = SPLIT_SM && FW < NW && fwave < 0;
        f32x4 s_cur[KB];
        bool act_cur = ntot > 0 && gstage_active(0);
        if constexpr (LATE_Q) {
            if (!act_cur) scale_q();
        }
        if (act_cur) {
            qk_preload(Kb0);
            qk_stage(Kb0, s_cur, std::integral_constant<bool, LATE_Q>{});
            if constexpr (CG > 1) xs_put(s_cur, 0);   // summed and masked after the barrier
            else mask_stage(s_cur, kb_of(0));
            if (early || sm_late) softmax_part(s_cur);
        }
        wait_vmcnt<0>();
        __syncthreads();   // V(0), K(1) resident; Kb0 free for K(2)
        auto step = [&](auto parity, int gs, auto early_c) {
            constexpr int P = decltype(parity)::value;
            constexpr bool EARLY = decltype(early_c)::value;
            float* k_fill = P ? Kb1 : Kb0;        // K(gs+2) -> buffer of K(gs)
            float* v_fill = P ? Vb0 : Vb1;        // V(gs+1)
            const float* k_next = P ? Kb0 : Kb1;  // K(gs+1)
            const float* v_cur = P ? Vb1 : Vb0;   // V(gs)
            const bool has_next = gs + 1 < ntot;
            if (gs + 2 < ntot) fill_stage(KL, Kh, kb_of(gs + 2), k_fill);
            if (has_next) fill_stage(VL, Vh, kb_of(gs + 1), v_fill);
            const bool switch_now = pairs && gs == nA - 1 && nB > 0;
            if (switch_now) load_q(q0_b + 16 * tile + li);
            const bool act_nxt = has_next && gstage_active(gs + 1);
            auto do_switch = [&]() {
                // block A's rows, full 128-bit stores (two_blocks needs d = D)
                const float lt = row4_sum(l);
                const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
                if (qrow < seq_q) {
                    float* orow = Oh + (size_t)qrow * D;
#pragma unroll
                    for (int hh = 0; hh < NVR; ++hh)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if constexpr (VW == 4) {
                                const f32x4 t = {o[4 * hh][r] * inv, o[4 * hh + 1][r] * inv,
                                                 o[4 * hh + 2][r] * inv, o[4 * hh + 3][r] * inv};
                                *reinterpret_cast<f32x4*>(orow + 64 * hh + VW * (4 * g + r)) = t;
                            } else {
                                const f32x2 t = {o[0][r] * inv, o[1][r] * inv};
                                *reinterpret_cast<f32x2*>(orow + VW * (4 * g + r)) = t;
                            }
                        }
                }
                q0 = q0_b;
                row_first = q0 + 16 * tile;
                qrow = row_first + li;
#pragma unroll
                for (int j = 0; j < NOB; ++j) o[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
                m = FA_NEG_INF;
                l = 0.0f;
                nref = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
                scale_q();
            };
            if constexpr (EARLY) {
                // This stage's PV (probabilities from the previous step; the
                // next K's first chunks are read during its last steps), then
                // the next stage's QK^T and softmax.
                if (act_cur) {
                    pv_preload(v_cur);
                    pv_part(s_cur, v_cur, [&](int step) {
                        if constexpr (PRE > 0) {
                            const int cc = step - (4 * KB - PRE);
                            if (act_nxt && cc >= 0 && cc < NC) k_chunk(k_next, cc, kpre[cc]);
                        }
                    });
                } else if (act_nxt) {
                    qk_preload(k_next);
                }
                if (switch_now) do_switch();
                if (act_nxt) {
                    qk_stage(k_next, s_cur, std::false_type{});
                    mask_stage(s_cur, kb_of(gs + 1));
                    softmax_part(s_cur);
                }
            } else {
                // This stage's softmax + PV, then the next stage's QK^T from
                // the other buffer, with no barrier between them.  Both stages
                // are resident: their first operands are read before the
                // softmax.  Column groups first sum the tile's partial scores
                // (slot P, written before the barrier that ended the last step).
                if constexpr (CG > 1) {
                    if (act_cur) {
                        xs_sum(s_cur, P);
                        mask_stage(s_cur, kb_of(gs));
                    }
                }
                if (act_cur) pv_preload(v_cur);
                if (act_nxt) qk_preload(k_next);
                if (act_cur) {
                    if (!sm_late) softmax_part(s_cur);
                    pv_part(s_cur, v_cur, no_hook);
                }
                if (switch_now) do_switch();
                if (act_nxt) {
                    qk_stage(k_next, s_cur, std::false_type{});
                    if constexpr (CG > 1) xs_put(s_cur, 1 - P);
                    else mask_stage(s_cur, kb_of(gs + 1));
                    if (sm_late) softmax_part(s_cur);
                }
            }
            if (has_next) {
                wait_vmcnt<0>();
                __syncthreads();
            }
            act_cur = act_nxt;
        };
        // One copy of the stage loop per order (a per-step branch between the
        // two orders leaves the register allocator spilling).
        auto run_steps = [&](auto early_c) {
            for (int gs = 0; gs < ntot; gs += 2) {
                step(std::integral_constant<int, 0>{}, gs, early_c);
                if (gs + 1 < ntot) step(std::integral_constant<int, 1>{}, gs + 1, early_c);
            }
        };
        if (early) run_steps(std::true_type{});
        else run_steps(std::false_type{});
    } else if constexpr (KVPP) {
        // One K buffer and one V buffer (src/v3.rs:445-483's overlap of the
        // next tile's loads with the current tile's work, with the buffers
        // taking turns): V(st) streams in by DMA while QK^T(st) reads K(st),
        // and K(st + 1) while softmax + PV(st) read V(st).  Two barriers per
        // stage, each after the DMA it waits for has had a compute phase to
        // land; the first also publishes the column groups' partial scores.
        if (nst > 0) fill_stage(KL, Kh, k0, Kb0);
        wait_vmcnt<0>();
        __syncthreads();
        for (int st = 0; st < nst; ++st) {
            const int kbase = k0 + st * SK;
            fill_stage(VL, Vh, kbase, Vb0);   // V buffer free: the last PV ended before the barrier
            const bool act = stage_active(st);
            f32x4 s[KB];
            if (act) {
                qk_preload(Kb0);
                qk_stage(Kb0, s, std::false_type{});
                xs_put(s, 0);
            }
            wait_vmcnt<0>();
            __syncthreads();   // V(st) resident, K buffer free, partial scores visible
            if (st + 1 < nst) fill_stage(KL, Kh, kbase + SK, Kb0);
            if (act) {
                xs_sum(s, 0);
                mask_stage(s, kbase);
                softmax_part(s);
                pv_preload(Vb0);
                pv_part(s, Vb0, no_hook);
            }
            wait_vmcnt<0>();
            __syncthreads();   // K(st + 1) resident, V buffer and score slots free
        }
    } else if constexpr (KV1) {
        // K and V of a stage in turn through the one buffer, each filled
        // through registers in two halves (a whole stage is 64 VGPRs per
        // lane): K, QK^T into the score slots, V, the softmax, PV.  Four
        // barriers per stage; the softmax runs while other waves store V.
        constexpr int HALF = LOAD_ITERS / 2;
        static_assert(LOAD_ITERS % 2 == 0, "stage fill in halves");
        auto fill_halves = [&](auto ld, const float* __restrict__ src, int kbase) {
            constexpr int LD = decltype(ld)::value;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                f32x4 rg[HALF];
#pragma unroll
                for (int it = 0; it < HALF; ++it) {
                    const int idx = tid + (h * HALF + it) * NT;
                    rg[it] = load4<LOADER != 0>(src, kbase + idx / CPR, seq_k, 4 * (idx % CPR), d);
                }
#pragma unroll
                for (int it = 0; it < HALF; ++it) {
                    const int idx = tid + (h * HALF + it) * NT;
                    *reinterpret_cast<f32x4*>(Kb0 + lds_off<LD>(idx / CPR, idx % CPR)) = rg[it];
                }
            }
        };
        for (int st = 0; st < nst; ++st) {
            const int kbase = k0 + st * SK;
            fill_halves(KL, Kh, kbase);
            __syncthreads();   // K(st) resident
            const bool act = stage_active(st);
            f32x4 s[KB];
            if (act) {
                qk_stage(Kb0, s, std::false_type{});
                xs_put(s, 0);
            }
            __syncthreads();   // K reads done, partial scores visible
            fill_halves(VL, Vh, kbase);
            if (act) {
                xs_sum(s, 0);
                mask_stage(s, kbase);
                softmax_part(s);
            }
            __syncthreads();   // V(st) resident
            if (act) pv_part(s, Kb0, no_hook);
            __syncthreads();   // buffer free for the next K
        }
    } else {
        // Single LDS stage; the next stage's global loads are issued into
        // registers before the current stage computes (D = 1024: its 64
        // registers would spill, so each stage is loaded when it is stored;
        // likewise the v1 split kernel with scalar loads at D = 256, which
        // spilled 5 VGPRs with the prefetch and needs 228 without it).
        constexpr bool PF = LOAD_ITERS <= 4 && !(STREAM && VARIANT == 1 && LOADER == 0 && D == 256);
        f32x4 kr[LOAD_ITERS], vr[LOAD_ITERS];
        if (PF && nst > 0) {
            load_regs(Kh, k0, kr);
            load_regs(Vh, k0, vr);
        }
        for (int st = 0; st < nst; ++st) {
            if (!PF) {
                load_regs(Kh, k0 + st * SK, kr);
                load_regs(Vh, k0 + st * SK, vr);
            }
            store_regs(KL, Kb0, kr);
            store_regs(VL, Vb0, vr);
            __syncthreads();
            if (PF && st + 1 < nst) {
                load_regs(Kh, k0 + (st + 1) * SK, kr);
                load_regs(Vh, k0 + (st + 1) * SK, vr);
            }
            const bool act = stage_active(st);
            f32x4 s[KB];
            if (act) {
                qk_preload(Kb0);
                pv_preload(Vb0);
                qk_stage(Kb0, s, std::false_type{});
                if constexpr (CG > 1) xs_put(s, 0);
            }
            if constexpr (CG > 1) __syncthreads();   // the tile's partial scores are in LDS
            if (act) {
                xs_sum(s, 0);
                mask_stage(s, k0 + st * SK);
                softmax_part(s);
                pv_part(s, Vb0, no_hook);
            }
            __syncthreads();
        }
    }

    if (splitk) {
        // Partial for this wave's 16-row tile and this key split, in the
        // split-KV layout fa_merge reads: O rows (unnormalised), m, l.
        const int qt = q0 / 16 + tile;
        if (qt >= p.nqt) return;
        // v2/v3: l is this lane's part of the row sum and o unnormalised; v1
        // keeps the row's full sum in l and o normalised by it (src/v1.rs:
        // 313-385), so its partial is o * l -- fa_merge then weighs the
        // normalised partials by l 2^(m - M) as it weighs v2's by 2^(m - M).
        const float lt = VARIANT == 1 ? l : row4_sum(l);
        if constexpr (VARIANT == 1) {
#pragma unroll
            for (int j = 0; j < NOB; ++j) o[j] *= lt;
        }
        // key split: slot (bh, qt, split); stream split: the block slot
        // (workgroup + global block index) times the block's 16-row tiles
        const size_t pidx = p.stream_per > 0 ? (size_t)ysplit * TILES + tile
                                             : ((size_t)bh * p.nqt + qt) * p.num_splits + ysplit;
        float* po = p.part_o + pidx * 16 * D;
        float* pml = p.part_ml + pidx * 32;
        if (g == 0 && cgrp == 0) {   // (m, l) agree across the column group
            pml[li] = m;
            pml[16 + li] = lt;
        }
        if constexpr (VW == 4 && CG == 1) {
            // D = 64, 128, 256: the tile in register order, each store a
            // contiguous 1 KB (64 lanes x 16 B): f32x4 (hh * 4 + r) * 64 +
            // lane holds columns 64 hh + 4 (4 g + r) .. + 3 of row li
            // (fa_merge_tiles reads this order).  Stored by rows instead,
            // every instruction wrote 16-byte pieces spread over 16 rows:
            // measured on config 5c (v3), 106.5 -> 101.1 us for the stream
            // split kernel with the merge.
            f32x4* pov = reinterpret_cast<f32x4*>(po);
#pragma unroll
            for (int hh = 0; hh < NVR; ++hh)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    pov[(hh * 4 + r) * 64 + lane] =
                        (f32x4){o[4 * hh][r], o[4 * hh + 1][r], o[4 * hh + 2][r], o[4 * hh + 3][r]};
            return;
        }
#pragma unroll
        for (int hh = 0; hh < NVR; ++hh)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int dv0 = c0 + 64 * hh + VW * (4 * g + r);
#pragma unroll
                for (int j = 0; j < VW; ++j) po[li * D + dv0 + j] = o[VW * hh + j][r];
            }
        return;
    }

    write_out();
}

// Stream split ("stream-K"): the (slice, query block, key stage) units of a
// v2/v3 prefill, slice-major and block-major, are cut into equal runs of
// p.stream_per units, one per workgroup, so every workgroup has the same
// number of stages however unequal the causal blocks are.  A run may end
// inside one block and start the next; each piece is a segment.  A block
// covered by one workgroup is written directly; a block shared by several
// gets one partial per workgroup and fa_merge combines them.  The partial of
// workgroup w for global block bg (slice * nqb + block) sits in block slot
// w + bg: a block's workgroups are consecutive and the last workgroup of a
// block is at most the first of the next, so slots never collide, and
// (workgroups + blocks - 1) slots of BQ rows hold them all.  Stage counts per block follow from
// BQ % SK == 0: block b has R (b + 1) stages (R = BQ / SK) while BQ (b + 1)
// <= seq_k (causal), otherwise ceil(seq_k / SK).
// Every unit index fits 32 bits (the host refuses plans whose unit total
// plus one run passes 2^31), so the quotients below are 32-bit unsigned
// divisions; products that can pass 2^32 on the way (b (b + 1)) are formed in
// 64 bits.  Measured (s_memtime in an instrumented copy, 16-bit causal config
// 2 on the stream split): with 64-bit divisions the decode of a workgroup's
// first segment took 3.6 us and of each later one 2.2 us.
struct StreamGeom {
    unsigned R, nsf, bf, u_head;
    bool causal;
};
__device__ __forceinline__ StreamGeom stream_geom(const FaParams& p, int bq, int sk_stage) {
    StreamGeom g;
    g.R = (unsigned)(bq / sk_stage);
    g.nsf = (unsigned)((p.seq_k + sk_stage - 1) / sk_stage);
    // blocks past the last query block do not exist: a key range longer than
    // the query range leaves every block on the triangle
    g.bf = (unsigned)min(p.seq_k / bq, p.nqb);
    g.causal = p.causal != 0 && !p.full_keys;   // v1: every block has all seq_k keys
    g.u_head = (unsigned)p.stream_head_units;
    return g;
}
// units of slice-local blocks 0 .. b-1 (b <= nqb: at most the slice's total)
__device__ __forceinline__ unsigned stream_prefix(const StreamGeom& g, unsigned b) {
    if (!g.causal) return b * g.nsf;
    if (b <= g.bf) return g.R * (unsigned)(((unsigned long long)b * (b + 1)) >> 1);
    return g.R * (unsigned)(((unsigned long long)g.bf * (g.bf + 1)) >> 1) + (b - g.bf) * g.nsf;
}
__device__ __forceinline__ unsigned stream_stages(const StreamGeom& g, unsigned b) {
    return (g.causal && b < g.bf) ? g.R * (b + 1) : g.nsf;
}
// the block holding slice-local unit r
__device__ __forceinline__ unsigned stream_block(const StreamGeom& g, unsigned r) {
    if (!g.causal) return r / g.nsf;
    const unsigned tri = stream_prefix(g, g.bf);
    if (r >= tri) return g.bf + (r - tri) / g.nsf;
    unsigned b = (unsigned)((sqrtf(8.0f * (float)(r / g.R) + 1.0f) - 1.0f) * 0.5f);
    while (b > 0 && stream_prefix(g, b) > r) --b;
    while (stream_prefix(g, b + 1) <= r) ++b;
    return b;
}
// workgroups first .. last share block b of slice h (units [ub, ub + n))
__device__ __forceinline__ void stream_span(const StreamGeom& g, unsigned per, unsigned h, unsigned b,
                                            unsigned& first, unsigned& last) {
    const unsigned ub = h * g.u_head + stream_prefix(g, b);
    first = ub / per;
    last = (ub + stream_stages(g, b) - 1) / per;
}

// The segments of this workgroup, run(seg) for each.  Split kernels
// (STREAM): the stream split's run of units (p.stream_per > 0), a loop over
// segments, or the key split's (block, split) from the compact grid.
// Otherwise one query block, or two-block pairs when PAIRS and the launch
// asks for them.  BQ rows per block, SK keys per stage.
template <int BQ, int SK, bool STREAM, bool PAIRS, typename F>
__device__ __forceinline__ void for_each_segment(const FaParams& p, F&& run) {
    static_assert(BQ % SK == 0, "stream split: whole stages per block");
    const bool stream = STREAM && p.stream_per > 0;
    // Loop state kept in SGPRs (readfirstlane): it is live across every
    // segment's stage loop, where VGPRs are short.  Unit indices fit 32 bits
    // (the host checks the total).
    unsigned u = 0, uend = 0, wg = 0;
    if (stream) {
        // Workgroups are dispatched round-robin over the 8 XCDs: consecutive
        // runs (mostly one slice's blocks) go to the same XCD, whose L2 then
        // holds that slice's K / V.
        const unsigned G = gridDim.x;
        const unsigned x = blockIdx.x;
        wg = (G % 8 == 0) ? (x % 8) * (G / 8) + x / 8 : x;
        const unsigned per = (unsigned)p.stream_per;
        u = wg * per;
        uend = min(u + per, (unsigned)p.bh * (unsigned)p.stream_head_units);
    }
    for (int it = 0;; ++it) {
        u = __builtin_amdgcn_readfirstlane(u);
        uend = __builtin_amdgcn_readfirstlane(uend);
        wg = __builtin_amdgcn_readfirstlane(wg);
        PrefillSeg seg{0, 0, -1, 0, -1, -1};
        if (stream) {
            if (u >= uend) break;
            const StreamGeom sg = stream_geom(p, BQ, SK);
            const unsigned h = u / sg.u_head, r = u - h * sg.u_head;
            const unsigned b = stream_block(sg, r);
            const unsigned s0 = r - stream_prefix(sg, b);
            const unsigned cnt = min(stream_stages(sg, b) - s0, uend - u);
            unsigned first, last;
            stream_span(sg, (unsigned)p.stream_per, h, b, first, last);
            seg.qb = (int)b;
            seg.bh = (int)h;
            seg.sbeg = (int)s0;
            seg.nst = (int)cnt;
            seg.slot = first == last ? -1 : (int)(wg + h * (unsigned)p.nqb + b);
            u += cnt;
        } else {
            if (it > 0) break;
            if (STREAM) {   // key split
                int y;
                map_block_split(p, seg.qb, seg.bh, y);
                seg.slot = y;
                seg.sbeg = y * (p.split_len / SK);
                seg.nst = p.split_len / SK;
            } else if (PAIRS && p.two_blocks != 0) {
                map_pair(p, blockIdx.x, seg.qb, seg.qb_second, seg.bh);
            } else {
                map_block(p, blockIdx.x, seg.qb, seg.bh);
            }
        }
        run(seg);
        if (stream) __syncthreads();   // LDS stages and slots are reused by the next segment
    }
}

// STREAM: the split instantiation (the stream split's loop over segments,
// or one key-split segment), which writes partials for fa_merge; the others
// run one unsplit segment, so their stage loops keep the registers that a
// loop around them, or the partial stores, would take.
template <int D, int VARIANT, int LOADER, bool STREAM>
__device__ __forceinline__ void prefill_body(const FaParams& p) {
    for_each_segment<fa_prefill_rows(D), fa_prefill_stage_keys(D, VARIANT), STREAM, VARIANT == 3 && D == 128>(
        p, [&](const PrefillSeg& seg) {
            // (the opaque tid spills at D >= 512 and is not needed there)
            prefill_segment<D, VARIANT, LOADER, STREAM, STREAM && D <= 256>(p, seg);
        });
}

// ---------------------------------------------------------------------------
// Split-KV decode kernel (new; no counterpart in the reference).
//
// For short query blocks against long key ranges.  Workgroup (split, qt, bh)
// (linearised split-fastest into blockIdx.x) takes keys [split*split_len, +split_len) of one (batch*head) for query rows
// 16qt .. 16qt+15 (zero-padded); its 4 waves take consecutive quarters.  A
// wave streams its keys 16 at a time straight from HBM with 128-bit loads
// into MFMA operand registers: S^T = K Q^T (K rows as the A operand, Q as B)
// and O^T += V^T P^T (V as A with the 64hh + 4i + j column map), with the
// same masked online softmax as the prefill kernel.  DBUF = true keeps two
// register sets so block n+1 is in flight while block n computes; DBUF =
// false re-issues each operand's loads as soon as it has been consumed.  The
// 4 waves merge through LDS into one partial (m, l, O) per workgroup, and
// fa_merge combines the splits by log-sum-exp.
// ---------------------------------------------------------------------------
// E: element type of Q/K/V (float, or bf16 / f16 widened to f32 as loaded).
// DBUF_REQ: double-buffer the K/V registers; D = 256 has no registers for it.
// KLDS (f32, 16-byte aligned operands, d % 4 == 0, D = 64, 128): K reaches
// the MFMA through LDS.  Each wave keeps a two-slot ring of its own 16-key
// blocks in LDS, filled by global->LDS DMA in whole padded rows (D + 8
// floats, written as 1 KiB runs: one wave-wide load covers about two
// contiguous K rows), and reads the A operand from there; V stays in
// registers.  The MFMA-layout K loads of the register path touch 16 rows x
// 64 bytes per instruction (measured: 5.7-6.1 TB/s for that pattern against
// 6.4-6.9 TB/s for whole rows).  No barriers: a wave only reads its own
// slots, after s_waitcnt on its own DMA.
// V1: v1's recurrence (src/v1.rs:291-385) -- the accumulator kept normalised,
// un-normalised by l * c before each block's PV and re-normalised by 1 / l
// after it -- and no causal skip: every key of the split is visited and
// masked, as v1 visits every tile.  The partial is un-normalised once at the
// end (o * l), so the waves' merge and fa_merge weigh it like v2's.
template <int D, bool VEC, bool DBUF_REQ, typename E = float, bool KLDS = false, bool V1 = false>
__device__ __forceinline__ void decode_body(const FaParams& p) {
    constexpr bool DBUF = DBUF_REQ && D <= 128;
    static_assert(!KLDS || (DBUF && VEC && D >= 64 && std::is_same<E, float>::value),
                  "LDS-staged K: f32, vector loads, 4 V columns per lane");
    constexpr int NQ = D / 4;          // MFMA k-steps over d (16x16x4)
    constexpr int NKL = D / 16;        // 128-bit K loads per lane per 16 keys
    constexpr int NVL = D / 64 > 0 ? D / 64 : 1;  // 128-bit V loads per lane per key step
    constexpr int VW = D >= 64 ? 4 : D / 16;      // floats per lane per V load
    constexpr int NOB = D / 16;        // O^T blocks of 16 dv
    constexpr int WSTRIDE = NOB * 4 * 64 + 128;
    constexpr int KLD = D + 8;                 // padded K row in LDS (floats)
    constexpr int KCH = KLD / 4;               // 16-byte chunks per padded row
    constexpr int KTOT = 16 * KCH;             // chunks per 16-key block image
    constexpr int KRUNS = (KTOT + 63) / 64;    // 1 KiB DMA runs per block
    constexpr int KIMG = KRUNS * 256;          // floats per wave slot (whole 1 KiB runs)
    static_assert(!KLDS || 4 * KIMG >= 3 * WSTRIDE, "merge area inside slot 0");
    __shared__ __attribute__((aligned(16))) float lds[KLDS ? 1 : 3 * WSTRIDE];
    __shared__ __attribute__((aligned(16))) float ks0[KLDS ? 4 * KIMG : 1];
    __shared__ __attribute__((aligned(16))) float ks1[KLDS ? 4 * KIMG : 1];
    float* const mlds = KLDS ? ks0 : lds;      // the waves' merge area

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lg = lane >> 4;          // lane group 0..3
    const int lr = lane & 15;

    // Workgroup x = split + num_splits * (qt + nqt * bh): a 1-D grid (any
    // number of slices), dispatched split-fastest as a 3-D grid would be.
    const int wgx = blockIdx.x;
    const int split = wgx % p.num_splits;
    const int tq = wgx / p.num_splits;
    const int qt = tq % p.nqt;
    const int bh = tq / p.nqt;
    const int seq_q = p.seq_q, seq_k = p.seq_k, d = p.d;
    const E* __restrict__ Qh = reinterpret_cast<const E*>(p.q) + (size_t)bh * seq_q * d;
    const E* __restrict__ Kh = reinterpret_cast<const E*>(p.k) + (size_t)bh * seq_k * d;
    const E* __restrict__ Vh = reinterpret_cast<const E*>(p.v) + (size_t)bh * seq_k * d;
    const float c = p.scale_log2e;
    const bool causal = p.causal != 0;

    const int q0 = qt * 16;
    const int qrow = q0 + lr;          // this lane's query (score column)
    const int qlast = min(seq_q, q0 + 16) - 1;

    // This wave's keys.  FA_DECODE_INTERLEAVE: wave w takes 16-key blocks
    // w, w + 4, ... of the split (the workgroup streams one contiguous region
    // of K and one of V); otherwise a contiguous quarter each.
#if FA_DECODE_INTERLEAVE
    const int kbeg = split * p.split_len + wave * 16;
    const int kstep = 64;
    int kend = min(seq_k, split * p.split_len + p.split_len);
#else
    const int wave_len = p.split_len / 4;
    const int kbeg = split * p.split_len + wave * wave_len;
    const int kstep = 16;
    int kend = min(seq_k, kbeg + wave_len);
#endif
    if (causal && !V1) kend = min(kend, qlast + 1);   // v2/v3: no key past the tile's last row

    // Q as the B operand: lane holds Q[qrow][16cc + 4lg + i] at qreg[4cc + i].
    float qreg[NQ];
#pragma unroll
    for (int cc = 0; cc < D / 16; ++cc) {
        const f32x4 t = widen<E>(load4r<E, VEC>(Qh, qrow, seq_q, 16 * cc + 4 * lg, d));
#pragma unroll
        for (int i = 0; i < 4; ++i) qreg[4 * cc + i] = t[i];
    }

    f32x4 o[NOB];
#pragma unroll
    for (int j = 0; j < NOB; ++j) o[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    float m = FA_NEG_INF, l = 0.0f;

    // K rows kb + lr (A operand), V rows kb + 4lg + r (A operand of O^T).
    typedef typename RawOf<E>::type R;
    auto load_k = [&](int kb, R* kk) {
#pragma unroll
        for (int cc = 0; cc < NKL; ++cc) kk[cc] = load4r<E, VEC, true>(Kh, kb + lr, kend, 16 * cc + 4 * lg, d);
    };
    auto load_v = [&](int kb, R* vv) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int hh = 0; hh < NVL; ++hh) {
                if constexpr (VW == 4) {
                    vv[r * NVL + hh] = load4r<E, VEC, true>(Vh, kb + 4 * lg + r, kend, 64 * hh + 4 * lr, d);
                } else {
                    // D = 32: 2 elements per lane (dv = 2*lr + j)
                    R t;
#pragma unroll
                    for (int e = 0; e < 4; ++e) t[e] = E(0.0f);
                    const int key = kb + 4 * lg + r;
                    if (key < kend) {
                        const E* vp = Vh + (size_t)key * d + VW * lr;
#pragma unroll
                        for (int e = 0; e < VW; ++e)
                            if (VW * lr + e < d) t[e] = vp[e];
                    }
                    vv[r * NVL + hh] = t;
                }
            }
    };

    // Scores of one 16-key block.  Blocked summation over d, 16 products
    // (4 MFMA steps) per block.
    auto scores = [&](int kb, const R* kk) -> f32x4 {
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int cc = 0; cc < NKL; ++cc) {
            f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
            const f32x4 kf = widen<E>(kk[cc]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                t = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[i], qreg[4 * cc + i], t, 0, 0, 0);
            s = (cc == 0) ? t : s + t;
        }
        return s;
    };
    // Masked online softmax + PV for one block (s[r] = score(key kb+4lg+r, qrow)).
    auto finish = [&](int kb, f32x4 s, const R* vv) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = kb + 4 * lg + r;
            if (key >= kend || (causal && key > qrow)) s[r] = FA_NEG_INF;
        }
        float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mt = row4_max(mt);
        const float m_new = fmaxf(m, mt);
        const float m_use = (m_new == FA_NEG_INF) ? 0.0f : m_new;
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[r] = fa_exp2((s[r] - m_use) * c);
            ps += s[r];
        }
        const float corr = rescale_factor(m, m_use, c);
        // v1: the row's full sum (its 4 lanes) every block; a block that
        // changes nothing (no visible key, same max) skips the round trip
        float inv = 1.0f;
        if constexpr (V1) {
            const float rs = row4_sum(ps);
            const float l_new = corr * l + rs;
            const bool moves = m_new != m || rs != 0.0f;
            const float f = moves ? l * corr : 1.0f;
#pragma unroll
            for (int j = 0; j < NOB; ++j) o[j] *= f;
            inv = !moves ? 1.0f : (l_new > 0.0f ? 1.0f / l_new : 0.0f);
            l = l_new;
        } else {
            l = corr * l + ps;
#pragma unroll
            for (int j = 0; j < NOB; ++j) o[j] *= corr;
        }
        m = m_new;
        // O^T[dv][q] += V^T P^T: block (hh, j) row i <-> dv = 64hh + VW*i + j
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int hh = 0; hh < NVL; ++hh) {
                const f32x4 vf = widen<E>(vv[r * NVL + hh]);
#pragma unroll
                for (int j = 0; j < VW; ++j)
                    o[hh * VW + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[j], s[r], o[hh * VW + j], 0, 0, 0);
            }
        if constexpr (V1) {
#pragma unroll
            for (int j = 0; j < NOB; ++j) o[j] *= inv;
        }
    };

    if constexpr (KLDS) {
        // Every load of the loop is a buffer load issued by all lanes (no
        // branches around loads), so the wave's vmcnt counts are exact and
        // the waits below name exactly the block they need.
        // Per-lane DMA offsets, the same for every block: image position
        // 64 i + lane is chunk pos % KCH of row pos / KCH (pad chunks and
        // columns past d fetch column 0); lanes past the image fetch out of
        // range (zeros) into the slot's slack after the image.
        int kvoff[KRUNS];
#pragma unroll
        for (int i = 0; i < KRUNS; ++i) {
            const int pos = 64 * i + lane;
            const int r = pos / KCH, ci = pos % KCH;
            const int col = (ci < D / 4 && 4 * ci < d) ? 4 * ci : 0;
            kvoff[i] = pos < KTOT ? 4 * (r * d + col) : 0x40000000;
        }
        // V (A operand of O^T): rows 4lg + r, columns 64hh + 4lr; columns
        // past d read out of range, as zeros (their O columns are not stored).
        int vvoff[4 * NVL];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int hh = 0; hh < NVL; ++hh)
                vvoff[r * NVL + hh] = 64 * hh + 4 * lr < d ? 4 * ((4 * lg + r) * d + 64 * hh + 4 * lr) : 0x40000000;
        // Block kb: K into a slot, V into registers.  The buffer ranges end at
        // kend, so rows past it read as zeros (masked to -inf in finish).
        auto load_block = [&](int kb, float* slot, R* vv) {
            const int bytes = min(16, kend - kb) * d * 4;
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(reinterpret_cast<const float*>(Kh) + (size_t)kb * d), (short)0, bytes, 0x00020000);
            const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(reinterpret_cast<const float*>(Vh) + (size_t)kb * d), (short)0, bytes, 0x00020000);
            float* dst = slot + wave * KIMG;
#pragma unroll
            for (int i = 0; i < KRUNS; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + 256 * i),
                                                         16, kvoff[i], 0, 0, FA_DECODE_KLDS_AUX);
#pragma unroll
            for (int j = 0; j < 4 * NVL; ++j)
                vv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, vvoff[j], 0, 2));
        };
        auto read_k = [&](const float* slot, R* kk) {
#pragma unroll
            for (int cc = 0; cc < NKL; ++cc)
                kk[cc] = *reinterpret_cast<const f32x4*>(slot + wave * KIMG + lr * KLD + 4 * (4 * cc + lg));
        };
        // DMA issued after a block's slot: its KRUNS runs and the 4 * NVL V loads
        constexpr int AFTER = KRUNS + 4 * NVL;
        R kk[NKL], va[4 * NVL], vb2[4 * NVL];
        int kb = kbeg;
        wait_vmcnt<0>();   // Q resident: the loop's waits then only concern blocks
        if (kb < kend) load_block(kb, ks0, va);
        while (kb < kend) {
            bool nx = kb + kstep < kend;
            if (nx) {
                load_block(kb + kstep, ks1, vb2);
                wait_vmcnt<AFTER>();
            } else {
                wait_vmcnt<0>();
            }
            read_k(ks0, kk);
            finish(kb, scores(kb, kk), va);
            kb += kstep;
            if (kb >= kend) break;
            nx = kb + kstep < kend;
            if (nx) {
                load_block(kb + kstep, ks0, va);
                wait_vmcnt<AFTER>();
            } else {
                wait_vmcnt<0>();
            }
            read_k(ks1, kk);
            finish(kb, scores(kb, kk), vb2);
            kb += kstep;
        }
    } else if constexpr (DBUF) {
        R ka[NKL], va[4 * NVL], kb2[NKL], vb2[4 * NVL];
        int kb = kbeg;
        if (kb < kend) {
            load_k(kb, ka);
            load_v(kb, va);
        }
        while (kb < kend) {
            if (kb + kstep < kend) {
                load_k(kb + kstep, kb2);
                load_v(kb + kstep, vb2);
            }
            finish(kb, scores(kb, ka), va);
            kb += kstep;
            if (kb >= kend) break;
            if (kb + kstep < kend) {
                load_k(kb + kstep, ka);
                load_v(kb + kstep, va);
            }
            finish(kb, scores(kb, kb2), vb2);
            kb += kstep;
        }
    } else {
        R kk[NKL], vv[4 * NVL];
        if (kbeg < kend) {
            load_k(kbeg, kk);
            load_v(kbeg, vv);
        }
        for (int kb = kbeg; kb < kend; kb += kstep) {
            const bool more = kb + kstep < kend;
            const f32x4 s = scores(kb, kk);
            if (more) load_k(kb + kstep, kk);   // K registers are free again
            finish(kb, s, vv);
            if (more) load_v(kb + kstep, vv);   // V registers are free again
        }
    }

    if constexpr (V1) {
        // l already holds the row's full sum; un-normalise the accumulator
#pragma unroll
        for (int j = 0; j < NOB; ++j) o[j] *= l;
    } else {
        l = row4_sum(l);
    }

    // Merge the 4 waves through LDS: waves 1..3 write, wave 0 combines (with
    // LDS-staged K, into slot 0 once every wave has read its last block).
    if constexpr (KLDS) __syncthreads();
    if (wave != 0) {
        float* w = mlds + (wave - 1) * WSTRIDE;
#pragma unroll
        for (int j = 0; j < NOB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) w[(j * 4 + r) * 64 + lane] = o[j][r];
        w[NOB * 4 * 64 + lane] = m;
        w[NOB * 4 * 64 + 64 + lane] = l;
    }
    __syncthreads();
    if (wave != 0) return;
    float mw[3];
    float mn = m;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
        mw[w] = mlds[w * WSTRIDE + NOB * 4 * 64 + lane];
        mn = fmaxf(mn, mw[w]);
    }
    const float mu = (mn == FA_NEG_INF) ? 0.0f : mn;
    const float c0 = rescale_factor(m, mu, c);
    l *= c0;
#pragma unroll
    for (int j = 0; j < NOB; ++j) o[j] *= c0;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
        const float cw = rescale_factor(mw[w], mu, c);
        l += mlds[w * WSTRIDE + NOB * 4 * 64 + 64 + lane] * cw;
#pragma unroll
        for (int j = 0; j < NOB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[j][r] += mlds[w * WSTRIDE + (j * 4 + r) * 64 + lane] * cw;
    }
    if (p.part_o == nullptr) {
        // One split (no workspace): the workgroup saw every key of its rows,
        // so it writes them normalised and no merge runs.
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        if (q0 + lr < seq_q) {
            float* orow = p.out + ((size_t)bh * seq_q + q0 + lr) * d;
#pragma unroll
            for (int hh = 0; hh < NVL; ++hh)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int dv0 = 64 * hh + VW * (4 * lg + r);
#pragma unroll
                    for (int j = 0; j < VW; ++j)
                        if (dv0 + j < d) orow[dv0 + j] = o[hh * VW + j][r] * inv;
                }
        }
        return;
    }
    // Partial for (bh, qt, split): O rows (unnormalised), m and l per query.
    const size_t pidx = ((size_t)bh * p.nqt + qt) * p.num_splits + split;
    float* po = p.part_o + pidx * 16 * D;
    float* pml = p.part_ml + pidx * 32;
    if (lg == 0) {
        pml[lr] = mn;
        pml[16 + lr] = l;
    }
    // lane holds O^T[dv][q = lr] for dv = 64hh + VW*(4lg + r) + j
#pragma unroll
    for (int hh = 0; hh < NVL; ++hh)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int dv0 = 64 * hh + VW * (4 * lg + r);
            if constexpr (VW == 4) {
                const f32x4 t = {o[hh * 4 + 0][r], o[hh * 4 + 1][r], o[hh * 4 + 2][r], o[hh * 4 + 3][r]};
                *reinterpret_cast<f32x4*>(po + lr * D + dv0) = t;
            } else {
#pragma unroll
                for (int j = 0; j < VW; ++j) po[lr * D + dv0 + j] = o[hh * VW + j][r];
            }
        }
}

// Combine the split partials of one query row (one wave per row):
// O = sum_s 2^((m_s - M) c) O_s / sum_s 2^((m_s - M) c) l_s, where empty
// splits (m_s = -inf, l_s = 0) weigh 0.
template <int D>
__device__ __forceinline__ void merge_body(const FaParams& p) {
    constexpr int CH = D / 4;                // 4-float column chunks per row
    constexpr int GROUPS = 64 / CH > 0 ? 64 / CH : 1;   // lanes sharing a chunk split the splits
    // FA_MERGE_ROWS rows per workgroup, one wave each with its own LDS area
    // (waves never wait for each other, so a wave may leave early).
    __shared__ float wts_all[FA_MERGE_ROWS][1024];
    __shared__ __attribute__((aligned(16))) float part_all[FA_MERGE_ROWS][64 * 4];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    float* const wts = wts_all[wave];
    float* const part = part_all[wave];
    const int row = blockIdx.x * FA_MERGE_ROWS + wave;   // bh * seq_q + q
    if (row >= p.bh * p.seq_q) return;
    // orders this wave's LDS writes before its reads of them (a wave's LDS
    // operations complete in order; this keeps the compiler from moving them)
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    const int q = row % p.seq_q, bh = row / p.seq_q;
    const int qt = q / 16, qi = q % 16;
    const float c = p.merge_scale;   // partial maxima -> log2 domain
    // Partial sp of this row's 16-row tile: pbase + sp * pstride.
    size_t pbase = ((size_t)bh * p.nqt + qt) * p.num_splits, pstride = 1;
    // Splits holding data for this row: all of them for split-KV; for the
    // prefill key split, those starting below the row's block key end.
    int ns = p.num_splits;
    if (p.stream_per > 0) {
        // stream split (split_len = the stage, ks_rows = the block): the
        // workgroups first .. last sharing this row's block (one: it wrote
        // the row), whose partials sit in block slots w + bh * nqb + block
        const StreamGeom sg = stream_geom(p, p.ks_rows, p.split_len);
        const int blk = q / p.ks_rows;
        unsigned first, last;
        stream_span(sg, (unsigned)p.stream_per, (unsigned)bh, (unsigned)blk, first, last);
        if (first == last) return;
        ns = (int)(last - first + 1);
        pstride = (size_t)(p.ks_rows / 16);
        pbase = ((size_t)first + (size_t)bh * p.nqb + blk) * pstride + (q % p.ks_rows) / 16;
    } else if (p.ks_rows > 0) {
        const int kend = (p.causal && !p.full_keys) ? min(p.seq_k, (q / p.ks_rows + 1) * p.ks_rows) : p.seq_k;
        ns = min(ns, (kend + p.split_len - 1) / p.split_len);
    }

    float M = FA_NEG_INF;
    for (int sp = lane; sp < ns; sp += 64) M = fmaxf(M, p.part_ml[(pbase + sp * pstride) * 32 + qi]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    const float Mu = (M == FA_NEG_INF) ? 0.0f : M;
    float L = 0.0f;
    for (int sp = lane; sp < ns; sp += 64) {
        const float* ml = p.part_ml + (pbase + sp * pstride) * 32;
        const float w = rescale_factor(ml[qi], Mu, c);
        wts[sp] = w;
        L += ml[16 + qi] * w;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) L += __shfl_xor(L, off);
    wave_sync();

    if constexpr (CH > 64) {
        // D > 256: each lane takes chunks lane, lane + 64, ...
        constexpr int CPL = CH / 64;
        const float* po = p.part_o + (pbase * 16 + qi) * D + 4 * lane;
        f32x4 acc[CPL];
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) acc[cc] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        for (int sp = 0; sp < ns; ++sp) {
            const float w = wts[sp];
#pragma unroll
            for (int cc = 0; cc < CPL; ++cc)
                acc[cc] += *reinterpret_cast<const f32x4*>(po + sp * pstride * 16 * D + 256 * cc) * w;
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        float* orow = p.out + (size_t)row * p.d;
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int col = 4 * (lane + 64 * cc) + e;
                if (col < p.d) orow[col] = acc[cc][e] * inv;
            }
        return;
    }
    const int ch = lane % CH, grp = lane / CH;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (grp < GROUPS) {
        const float* po = p.part_o + (pbase * 16 + qi) * D + 4 * ch;
#pragma unroll 8
        for (int sp = grp; sp < ns; sp += GROUPS)
            acc += *reinterpret_cast<const f32x4*>(po + sp * pstride * 16 * D) * wts[sp];
    }
    if constexpr (GROUPS > 1) {
        *reinterpret_cast<f32x4*>(part + 4 * lane) = acc;
        wave_sync();
        if (grp != 0) return;
        for (int g2 = 1; g2 < GROUPS; ++g2) acc += *reinterpret_cast<const f32x4*>(part + 4 * (g2 * CH + ch));
    }
    if (lane >= CH) return;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    float* orow = p.out + (size_t)row * p.d;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (4 * ch + e < p.d) orow[4 * ch + e] = acc[e] * inv;
}

// fa_merge_tiles: the log-sum-exp merge of the f32 prefill key split and
// stream split at D = 64, 128, 256, whose partials are 16-row tiles in
// register order (prefill_segment: f32x4 (hh * 4 + r) * 64 + lane holds
// columns 64 hh + 4 (4 g + r) .. + 3 of row li = lane % 16, g = lane / 16).
// One workgroup per (slice, 16-row tile), one wave per 64-column group hh:
// every load is a contiguous 1 KB, and the rows are stored 64 contiguous
// bytes at a time (lane_group_transpose4).  The splits of a tile, their slots and the weights 2^((m - M) c)
// are those of merge_body, taken row by row in each lane.
template <int D>
__device__ __forceinline__ void merge_tiles_body(const FaParams& p) {
    static_assert(D == 64 || D == 128 || D == 256, "register-order tiles: D = 64, 128, 256");
    const int lane = threadIdx.x & 63;
    const int hh = threadIdx.x >> 6;    // the wave's 64-column group
    const int li = lane & 15, g = lane >> 4;
    const int bh = blockIdx.x / p.nqt, qt = blockIdx.x % p.nqt;
    if (bh >= p.bh) return;
    const int q0 = 16 * qt;
    const float c = p.merge_scale;
    size_t pbase = ((size_t)bh * p.nqt + qt) * p.num_splits, pstride = 1;
    int ns = p.num_splits;
    if (p.stream_per > 0) {
        const StreamGeom sg = stream_geom(p, p.ks_rows, p.split_len);
        const int blk = q0 / p.ks_rows;
        unsigned first, last;
        stream_span(sg, (unsigned)p.stream_per, (unsigned)bh, (unsigned)blk, first, last);
        if (first == last) return;   // one workgroup wrote the block's rows
        ns = (int)(last - first + 1);
        pstride = (size_t)(p.ks_rows / 16);
        pbase = ((size_t)first + (size_t)bh * p.nqb + blk) * pstride + (q0 % p.ks_rows) / 16;
    } else {
        const int kend = (p.causal && !p.full_keys) ? min(p.seq_k, (q0 / p.ks_rows + 1) * p.ks_rows) : p.seq_k;
        ns = min(ns, (kend + p.split_len - 1) / p.split_len);
    }
    float M = FA_NEG_INF;
    for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, p.part_ml[(pbase + sp * pstride) * 32 + li]);
    const float Mu = (M == FA_NEG_INF) ? 0.0f : M;
    float L = 0.0f;
    f32x4 acc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 2
    for (int sp = 0; sp < ns; ++sp) {
        const size_t slot = pbase + sp * pstride;
        const float* ml = p.part_ml + slot * 32;
        const float w = rescale_factor(ml[li], Mu, c);
        L += ml[16 + li] * w;
        const f32x4* po = reinterpret_cast<const f32x4*>(p.part_o + slot * 16 * D) + hh * 4 * 64 + lane;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] += po[r * 64] * w;
    }
    const int row = q0 + li;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    // row order (every lane takes part in the swaps): columns 64 hh + 16 r +
    // 4 g, 64 contiguous bytes of every row per store (config 5c: ~0.3 us)
    float v[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[r][e] = acc[r][e] * inv;
    lane_group_transpose4(v);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = (f32x4){v[r][0], v[r][1], v[r][2], v[r][3]};
    if (row >= p.seq_q) return;
    float* orow = p.out + ((size_t)bh * p.seq_q + row) * p.d;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int dv0 = 64 * hh + 16 * r + 4 * g;
        // 128-bit stores where the output allows them (the split kernels
        // also serve unaligned outputs and d % 4 != 0 through scalar loads)
        if (dv0 + 4 <= p.d && (reinterpret_cast<uintptr_t>(orow + dv0) & 15) == 0) {
            *reinterpret_cast<f32x4*>(orow + dv0) = acc[r];
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (dv0 + e < p.d) orow[dv0 + e] = acc[r][e];
        }
    }
}

#include "fa_decode_rows.inc"

// ---------------------------------------------------------------------------
// Heads wider than 2048 columns (the crate's flash path takes any d_head,
// src/v2.rs:175-189, with an O(Br x d) accumulator per query block): one
// workgroup of NW = 8 waves per 16-row query tile, the unnormalised O
// accumulator kept in `out` itself (the tile's rows of the caller's [seq_q, d]
// output), and Q, K and V read from global memory (L2) straight into MFMA
// operands -- no LDS staging, since each wave reads its own columns.  Per
// stage of 64 keys:
//  1. each wave forms partial scores S^T over its 64-column chunks (chunk
//     ch = wave, wave + NW, ...; a fresh 16-MFMA chain per chunk, added to
//     the wave's running sum), and the NW partials are summed through LDS
//     in wave order, so every wave holds bit-identical scores;
//  2. every wave runs the same online softmax with the exact running max
//     (src/v2.rs:289-372);
//  3. each wave reads its chunks of O from `out`, rescales them, adds
//     V^T P^T and writes them back (lane l owns query row l % 16 and the 16
//     consecutive columns 16 (l / 16) .. +15 of each chunk).
// v1 keeps O normalised at every stage (src/v1.rs:313-385) and visits every
// key; v2 / v3 stop at the tile's causal end and normalise in the last stage
// (v3's double-buffered LDS stages have nothing to stage here: v3 runs v2's
// steps).  Columns past d and rows past seq_q / seq_k read as zeros and are
// never written.
// ---------------------------------------------------------------------------
// NCR > 0 (heads of at most NW * NCR * 64 columns): each wave keeps its NCR
// chunks of O in registers for the whole kernel instead -- no read-modify-
// write of `out` per stage -- and writes them once at the end.
template <int VARIANT, bool VEC, int NCR>
__device__ __forceinline__ void prefill_any_body(const FaParams& p) {
    constexpr int NW = 8;          // waves (column-chunk owners)
    constexpr int SK = 64;         // keys per stage
    constexpr int KB = SK / 16;    // 16-key blocks per stage
    constexpr int CW = 64;         // columns per chunk
    // partial scores of every wave, two slots (one barrier per stage)
    __shared__ __attribute__((aligned(16))) f32x4 Xs[2][NW][KB][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, li = lane & 15;
    int qt, bh;
    map_block(p, blockIdx.x, qt, bh);   // p.nqb: 16-row tiles per slice
    const int seq_q = p.seq_q, seq_k = p.seq_k, d = p.d;
    const float* __restrict__ Qh = p.q + (size_t)bh * seq_q * d;
    const float* __restrict__ Kh = p.k + (size_t)bh * seq_k * d;
    const float* __restrict__ Vh = p.v + (size_t)bh * seq_k * d;
    float* __restrict__ Oh = p.out + (size_t)bh * seq_q * d;
    const int row0 = qt * 16, qrow = row0 + li;
    const bool row_ok = qrow < seq_q;
    const bool causal = p.causal != 0;
    const float c = p.scale_log2e;
    // v1 visits every key (src/v1.rs:209-216); v2 / v3 stop after the
    // tile's last row (src/v2.rs:208-212)
    const int kend = (VARIANT != 1 && causal) ? min(seq_k, row0 + 16) : seq_k;
    const int nst = (kend + SK - 1) / SK;
    const int nch = (d + CW - 1) / CW;
    float* const orow = Oh + (size_t)qrow * d;

    // O chunk of this lane: o[j][r] = O[qrow][col0 + 16 g + 4 r + j]
    auto load_o = [&](int col0, f32x4* o) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const f32x4 t = load4<VEC>(Oh, qrow, seq_q, col0 + 16 * g + 4 * r, d);
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j][r] = t[j];
        }
    };
    auto store_o = [&](int col0, const f32x4* o) {
        if (!row_ok) return;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int col = col0 + 16 * g + 4 * r;
            if (VEC && col < d) {
                *reinterpret_cast<f32x4*>(orow + col) = (f32x4){o[0][r], o[1][r], o[2][r], o[3][r]};
            } else if (!VEC) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (col + j < d) orow[col + j] = o[j][r];
            }
        }
    };

    float m = FA_NEG_INF;   // running max of the row's log2-domain scores
    float l = 0.0f;         // running row sum (v1: of the normalised accumulator)
    f32x4 oreg[NCR > 0 ? NCR : 1][4];   // register-held chunks: ch = wave + NW j
#pragma unroll
    for (int j = 0; j < (NCR > 0 ? NCR : 1); ++j)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) oreg[j][jj] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // O^T += V^T P^T for one chunk (64 columns from col0) over the stage's keys
    auto pv_chunk = [&](const f32x4* s_, int kbase, int col0, f32x4* o) {
#pragma unroll
        for (int step = 0; step < 4 * KB; ++step) {
            const int key = kbase + 16 * (step / 4) + 4 * g + (step % 4);
            const f32x4 vv = load4<VEC>(Vh, key, seq_k, col0 + 4 * li, d);
            const float pr = s_[step / 4][step % 4];
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[j], pr, o[j], 0, 0, 0);
        }
    };
    for (int st = 0; st < nst; ++st) {
        const int kbase = st * SK;
        const int slot = st & 1;
        // 1. this wave's partial scores
        f32x4 s[KB];
#pragma unroll
        for (int b = 0; b < KB; ++b) s[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        for (int ch = wave; ch < nch; ch += NW) {
            f32x4 t[KB];
#pragma unroll
            for (int b = 0; b < KB; ++b) t[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int cc = 0; cc < CW / 16; ++cc) {
                const int col = ch * CW + 16 * cc + 4 * g;
                const f32x4 qv = load4<VEC>(Qh, qrow, seq_q, col, d);
                f32x4 kv[KB];
#pragma unroll
                for (int b = 0; b < KB; ++b) kv[b] = load4<VEC>(Kh, kbase + 16 * b + li, seq_k, col, d);
#pragma unroll
                for (int b = 0; b < KB; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) t[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[b][i], qv[i], t[b], 0, 0, 0);
            }
#pragma unroll
            for (int b = 0; b < KB; ++b) s[b] += t[b];
        }
#pragma unroll
        for (int b = 0; b < KB; ++b) Xs[slot][wave][b][lane] = s[b];
        __syncthreads();
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            f32x4 x = Xs[slot][0][b][lane];
#pragma unroll
            for (int w = 1; w < NW; ++w) x += Xs[slot][w][b][lane];
            s[b] = x;
        }
        // 2. online softmax: scores in the log2 domain (dot * scale * log2 e),
        // keys past seq_k and, causal, past the row masked (top-left aligned,
        // src/naive.rs:37)
        float mt = FA_NEG_INF;
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kbase + 16 * b + 4 * g + r;
                const float x = (key >= seq_k || (causal && key > qrow)) ? FA_NEG_INF : s[b][r] * c;
                s[b][r] = x;
                mt = fmaxf(mt, x);
            }
        mt = row4_max(mt);
        const float m_new = fmaxf(m, mt);
        const float corr = rescale_factor(m, m_new, 1.0f);   // 0 while the row has seen no key
        const float mref = (m_new == FA_NEG_INF) ? 0.0f : m_new;
        float ps = 0.0f;
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[b][r] = fa_exp2(s[b][r] - mref);
                ps += s[b][r];
            }
        const float rs = row4_sum(ps);
        const float l_new = l * corr + rs;
        const bool last = NCR == 0 && st + 1 == nst;   // register-held O is normalised at the end
        // factors on the stored O before and after this stage's PV
        float f_pre, f_post;
        bool moves = true;
        if (VARIANT == 1) {
            // un-normalise by l * corr, add PV, re-normalise by 1 / l_new;
            // a stage that adds nothing to the row and does not move its max
            // is an identity and is skipped (no rounding drift)
            moves = m_new != m || rs != 0.0f;
            f_pre = l * corr;
            f_post = l_new > 0.0f ? 1.0f / l_new : 0.0f;
        } else {
            f_pre = corr;
            f_post = last ? (l_new > 0.0f ? 1.0f / l_new : 0.0f) : 1.0f;
        }
        m = m_new;
        l = l_new;
        // 3. this wave's chunks of O (the whole wave skips when no row moves)
        if (__builtin_amdgcn_ballot_w64(moves) != 0) {
            if constexpr (NCR > 0) {
                // rows that do not move keep their accumulator as it is
                const float fa = moves ? f_pre : 1.0f;
                const float fb = moves ? f_post : 1.0f;
#pragma unroll
                for (int j = 0; j < NCR; ++j) {
                    if (wave + NW * j < nch) {
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj) oreg[j][jj] *= fa;
                        pv_chunk(s, kbase, (wave + NW * j) * CW, oreg[j]);
                        if (VARIANT == 1) {
#pragma unroll
                            for (int jj = 0; jj < 4; ++jj) oreg[j][jj] *= fb;
                        }
                    }
                }
            } else {
                for (int ch = wave; ch < nch; ch += NW) {
                    const int col0 = ch * CW;
                    f32x4 o[4];
                    if (st == 0 || !row_ok) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) o[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
                    } else {
                        load_o(col0, o);
#pragma unroll
                        for (int j = 0; j < 4; ++j) o[j] *= f_pre;
                    }
                    pv_chunk(s, kbase, col0, o);
                    if (VARIANT == 1 || last) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) o[j] *= f_post;
                    }
                    if (moves) store_o(col0, o);
                }
            }
        }
    }
    if constexpr (NCR > 0) {
        // v2 / v3: the final normalisation; v1's accumulator is normalised
        const float inv = VARIANT == 1 ? 1.0f : (l > 0.0f ? 1.0f / l : 0.0f);
#pragma unroll
        for (int j = 0; j < NCR; ++j) {
            if (wave + NW * j < nch) {
                f32x4 o[4];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) o[jj] = oreg[j][jj] * inv;
                store_o((wave + NW * j) * CW, o);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Naive attention: the textbook three passes over a materialised score
// matrix (src/naive.rs:14-75), kept as an on-device reference -- in f32 as
// the crate computes it, or in f64 to check the fast kernels on shapes too
// large for a CPU oracle.  Scores and probabilities live in one
// [heads, seq_q, seq_k] buffer of T.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T naive_scale(const NaiveParams& p);
template <>
__device__ __forceinline__ float naive_scale<float>(const NaiveParams& p) { return p.scale_f; }
template <>
__device__ __forceinline__ double naive_scale<double>(const NaiveParams& p) { return p.scale_d; }

__device__ __forceinline__ float naive_exp(float x) { return expf(x); }
__device__ __forceinline__ double naive_exp(double x) { return exp(x); }

// S[i][j] = (q_i . k_j) * scale, -inf where causal && j > i
// (src/naive.rs:33-44).  64x64 tile per 256-thread workgroup, 4x4 per
// thread (rows ty + 16x, columns tx + 16y), d in chunks of 16 through LDS.
template <typename T>
__device__ __forceinline__ void naive_scores_body(const NaiveParams& p) {
    constexpr int TM = 64, TK = 16;
    __shared__ T Qs[TK][TM + 1];
    __shared__ T Ks[TK][TM + 1];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int j0 = blockIdx.x * TM, i0 = blockIdx.y * TM, h = blockIdx.z;
    const int sq = p.seq_q, sk = p.seq_k, d = p.d;
    const float* __restrict__ Q = p.q + (size_t)h * sq * d;
    const float* __restrict__ K = p.k + (size_t)h * sk * d;
    T* __restrict__ S = static_cast<T*>(p.s) + (size_t)h * sq * sk;
    T acc[4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = T(0);
    const bool all_future = p.causal && j0 > i0 + TM - 1;   // every score of the tile is masked
    if (!all_future) {
        for (int kc = 0; kc < d; kc += TK) {
            for (int e = threadIdx.x; e < TM * TK; e += 256) {
                const int r = e / TK, c = e % TK, dc = kc + c;
                Qs[c][r] = (i0 + r < sq && dc < d) ? T(Q[(size_t)(i0 + r) * d + dc]) : T(0);
                Ks[c][r] = (j0 + r < sk && dc < d) ? T(K[(size_t)(j0 + r) * d + dc]) : T(0);
            }
            __syncthreads();
#pragma unroll
            for (int c = 0; c < TK; ++c) {
                T a[4], b[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    a[x] = Qs[c][ty + 16 * x];
                    b[x] = Ks[c][tx + 16 * x];
                }
#pragma unroll
                for (int x = 0; x < 4; ++x)
#pragma unroll
                    for (int y = 0; y < 4; ++y) acc[x][y] = fma(a[x], b[y], acc[x][y]);
            }
            __syncthreads();
        }
    }
    const T scale = naive_scale<T>(p);
    const T ninf = -__builtin_huge_val();
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        const int i = i0 + ty + 16 * x;
        if (i >= sq) continue;
#pragma unroll
        for (int y = 0; y < 4; ++y) {
            const int j = j0 + tx + 16 * y;
            if (j < sk) S[(size_t)i * sk + j] = (p.causal && j > i) ? ninf : acc[x][y] * scale;
        }
    }
}

// Row softmax in place (src/naive.rs:46-59): max, exp(s - max) and its sum,
// then multiply by (sum > 0 ? 1/sum : 0).  One 256-thread workgroup per row.
template <typename T>
__device__ __forceinline__ T naive_block_reduce(T v, bool is_max, T* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const T o = __shfl_xor(v, off);
        v = is_max ? (o > v ? o : v) : v + o;
    }
    const int wave = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    T r = red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) r = is_max ? (red[w] > r ? red[w] : r) : r + red[w];
    __syncthreads();
    return r;
}

template <typename T>
__device__ __forceinline__ void naive_softmax_body(const NaiveParams& p) {
    __shared__ T red[4];
    const int sk = p.seq_k;
    T* __restrict__ s = static_cast<T*>(p.s) + (size_t)blockIdx.x * sk;   // row (head, i) of this chunk
    T m = -__builtin_huge_val();
    for (int j = threadIdx.x; j < sk; j += 256) m = s[j] > m ? s[j] : m;
    m = naive_block_reduce<T>(m, true, red);
    T sum = T(0);
    for (int j = threadIdx.x; j < sk; j += 256) {
        const T e = naive_exp(s[j] - m);
        s[j] = e;
        sum += e;
    }
    sum = naive_block_reduce<T>(sum, false, red);
    const T inv = sum > T(0) ? T(1) / sum : T(0);
    for (int j = threadIdx.x; j < sk; j += 256) s[j] *= inv;
}

// out[i][c] = sum_j P[i][j] V[j][c], skipping p == 0 (src/naive.rs:61-74);
// with causal masking P is exactly 0 past the tile's last row, so those keys
// are not visited.  64 rows x 64 columns per workgroup, keys in chunks of 16.
template <typename T>
__device__ __forceinline__ void naive_pv_body(const NaiveParams& p) {
    constexpr int TM = 64, TK = 16;
    __shared__ T Ps[TK][TM + 1];
    __shared__ T Vs[TK][TM + 1];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int c0 = blockIdx.x * TM, i0 = blockIdx.y * TM, h = blockIdx.z;
    const int sq = p.seq_q, sk = p.seq_k, d = p.d;
    const T* __restrict__ P = static_cast<const T*>(p.s) + (size_t)h * sq * sk;
    const float* __restrict__ V = p.v + (size_t)h * sk * d;
    float* __restrict__ O = p.out + (size_t)h * sq * d;
    T acc[4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = T(0);
    const int jend = p.causal ? min(sk, i0 + TM) : sk;
    for (int jc = 0; jc < jend; jc += TK) {
        for (int e = threadIdx.x; e < TM * TK; e += 256) {
            const int r = e / TK, c = e % TK;          // P: row r, key c
            Ps[c][r] = (i0 + r < sq && jc + c < sk) ? P[(size_t)(i0 + r) * sk + jc + c] : T(0);
            const int kk = e / TM, cc = e % TM;        // V: key kk, column cc
            Vs[kk][cc] = (jc + kk < sk && c0 + cc < d) ? T(V[(size_t)(jc + kk) * d + c0 + cc]) : T(0);
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < TK; ++c) {
            T a[4], b[4];
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                a[x] = Ps[c][ty + 16 * x];
                b[x] = Vs[c][tx + 16 * x];
            }
#pragma unroll
            for (int x = 0; x < 4; ++x)
#pragma unroll
                for (int y = 0; y < 4; ++y) acc[x][y] = a[x] != T(0) ? fma(a[x], b[y], acc[x][y]) : acc[x][y];
        }
        __syncthreads();
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        const int i = i0 + ty + 16 * x;
        if (i >= sq) continue;
#pragma unroll
        for (int y = 0; y < 4; ++y) {
            const int c = c0 + tx + 16 * y;
            if (c < d) O[(size_t)i * d + c] = static_cast<float>(acc[x][y]);
        }
    }
}

// ---------------------------------------------------------------------------
// Named entry points for hipModuleGetFunction.
// ---------------------------------------------------------------------------
// fa_prefill_v{V}_d{D}_{L}: L = 0 scalar loads, 1 vector loads, 2 LDS DMA (v3);
// fa_prefill_v{V}_d{D}_{L}s: the split instantiation (stream split and key
// split; v1 keeps its per-stage normalisation and visits every key).
#define FA_PREFILL(D, VAR, LD)                                                                   \
    extern "C" __global__ void __launch_bounds__(64 * fa_prefill_waves(D), 8 / fa_prefill_waves(D))   \
        fa_prefill_v##VAR##_d##D##_##LD(FaParams p) {                                                \
        prefill_body<D, VAR, LD, false>(p);                                                      \
    }
#define FA_PREFILL_S(D, VAR, LD)                                                                 \
    extern "C" __global__ void __launch_bounds__(64 * fa_prefill_waves(D), 8 / fa_prefill_waves(D))   \
        fa_prefill_v##VAR##_d##D##_##LD##s(FaParams p) {                                             \
        prefill_body<D, VAR, LD, true>(p);                                                       \
    }
#define FA_PREFILL_ALL(D)  \
    FA_PREFILL(D, 1, 0)    \
    FA_PREFILL(D, 1, 1)    \
    FA_PREFILL_S(D, 1, 0)  \
    FA_PREFILL_S(D, 1, 1)  \
    FA_PREFILL(D, 2, 0)    \
    FA_PREFILL(D, 2, 1)    \
    FA_PREFILL(D, 3, 0)    \
    FA_PREFILL(D, 3, 1)    \
    FA_PREFILL(D, 3, 2)    \
    FA_PREFILL_S(D, 2, 0)  \
    FA_PREFILL_S(D, 2, 1)  \
    FA_PREFILL_S(D, 3, 0)  \
    FA_PREFILL_S(D, 3, 1)  \
    FA_PREFILL_S(D, 3, 2)

FA_PREFILL_ALL(32)
FA_PREFILL_ALL(64)
FA_PREFILL_ALL(128)
FA_PREFILL_ALL(256)
FA_PREFILL_ALL(512)
// D = 1024: one K + V stage fills the LDS; v3's DMA loader alternates the K
// and V buffers (its scalar / 128-bit loaders run v2's single-stage schedule)
FA_PREFILL(1024, 1, 0)
FA_PREFILL(1024, 1, 1)
FA_PREFILL(1024, 2, 0)
FA_PREFILL(1024, 2, 1)
FA_PREFILL(1024, 3, 0)
FA_PREFILL(1024, 3, 1)
FA_PREFILL(1024, 3, 2)
FA_PREFILL_S(1024, 1, 0)
FA_PREFILL_S(1024, 1, 1)
FA_PREFILL_S(1024, 2, 0)
FA_PREFILL_S(1024, 2, 1)
FA_PREFILL_S(1024, 3, 0)
FA_PREFILL_S(1024, 3, 1)
FA_PREFILL_S(1024, 3, 2)
// D = 2048 (heads of 1025..2048 columns): column groups of 8 waves per
// 16-row tile; K and V share one LDS buffer; v3 runs v2's schedule
#define FA_PREFILL_2048(VAR) FA_PREFILL(2048, VAR, 0) FA_PREFILL(2048, VAR, 1) \
    FA_PREFILL_S(2048, VAR, 0) FA_PREFILL_S(2048, VAR, 1)
FA_PREFILL_2048(1)
FA_PREFILL_2048(2)
FA_PREFILL_2048(3)
// Heads wider than 2048 columns: fa_prefill_v{V}_dany_{L} (any d, O in the
// output rows) and fa_prefill_v{V}_dreg_{L} (d <= 4096, O in registers);
// L = 0 scalar loads (any d), 1 vector loads (d % 4 == 0, 16-byte aligned
// operands)
#define FA_PREFILL_ANY(VAR, LD)                                                                  \
    extern "C" __global__ void __launch_bounds__(512, 2) fa_prefill_v##VAR##_dany_##LD(FaParams p) {  \
        prefill_any_body<VAR, LD != 0, 0>(p);                                                    \
    }                                                                                            \
    extern "C" __global__ void __launch_bounds__(512, 1) fa_prefill_v##VAR##_dreg_##LD(FaParams p) {  \
        prefill_any_body<VAR, LD != 0, 8>(p);                                                    \
    }
FA_PREFILL_ANY(1, 0)
FA_PREFILL_ANY(1, 1)
FA_PREFILL_ANY(2, 0)
FA_PREFILL_ANY(2, 1)
FA_PREFILL_ANY(3, 0)
FA_PREFILL_ANY(3, 1)

// Decode register double-buffering (FA_DECODE_DBUF=1) trades occupancy for
// one block of loads in flight per register set.
#ifndef FA_DECODE_DBUF
#define FA_DECODE_DBUF 1
#endif
#define FA_DECODE(D, VEC, OCC1, OCC2)                                                            \
    extern "C" __global__ void __launch_bounds__(256, FA_DECODE_DBUF ? OCC2 : OCC1)              \
        fa_decode_d##D##_##VEC(FaParams p) {                                                     \
        decode_body<D, VEC != 0, FA_DECODE_DBUF != 0>(p);                                        \
    }
FA_DECODE(32, 1, 4, 4)
FA_DECODE(32, 0, 4, 4)
FA_DECODE(64, 1, 4, 3)
FA_DECODE(64, 0, 4, 3)
FA_DECODE(128, 1, 3, 2)
FA_DECODE(128, 0, 3, 2)
FA_DECODE(256, 1, 1, 1)
FA_DECODE(256, 0, 1, 1)
// fa_decode_d{D}_2: K staged through per-wave LDS rings by DMA (f32, D = 64, 128)
#define FA_DECODE_KLDS(D)                                                                         \
    extern "C" __global__ void __launch_bounds__(256, 2) fa_decode_d##D##_2(FaParams p) {         \
        decode_body<D, true, true, float, true>(p);                                               \
    }
FA_DECODE_KLDS(64)
FA_DECODE_KLDS(128)
// fa_decode_v1_d{D}_{L}: v1's per-block normalisation, every key visited.
// D = 128 with scalar loads re-issues each operand's loads once consumed (no
// register double buffer): with it the kernel spilled 32 VGPRs.
#define FA_DECODE_V1(D, VEC, DBUF, OCC)                                                          \
    extern "C" __global__ void __launch_bounds__(256, OCC) fa_decode_v1_d##D##_##VEC(FaParams p) { \
        decode_body<D, VEC != 0, DBUF, float, false, true>(p);                                   \
    }
FA_DECODE_V1(32, 1, true, 4)
FA_DECODE_V1(32, 0, true, 4)
FA_DECODE_V1(64, 1, true, 3)
FA_DECODE_V1(64, 0, true, 3)
FA_DECODE_V1(128, 1, true, 2)
FA_DECODE_V1(128, 0, false, 2)
FA_DECODE_V1(256, 1, false, 1)
FA_DECODE_V1(256, 0, false, 1)
#define FA_DECODE_KLDS_V1(D)                                                                      \
    extern "C" __global__ void __launch_bounds__(256, 2) fa_decode_v1_d##D##_2(FaParams p) {      \
        decode_body<D, true, true, float, true, true>(p);                                         \
    }
FA_DECODE_KLDS_V1(64)
FA_DECODE_KLDS_V1(128)

// fa_decode_{bf16,f16}_d{D}_{VEC}: 16-bit Q/K/V widened to f32 as loaded.
#define FA_DECODE_LP(D, TN, T, VEC, OCC1, OCC2)                                                   \
    extern "C" __global__ void __launch_bounds__(256, FA_DECODE_DBUF ? OCC2 : OCC1)              \
        fa_decode_##TN##_d##D##_##VEC(FaParams p) {                                              \
        decode_body<D, VEC != 0, FA_DECODE_DBUF != 0, T>(p);                                     \
    }
#define FA_DECODE_LP_ALL(TN, T)              \
    FA_DECODE_LP(32, TN, T, 1, 4, 4)         \
    FA_DECODE_LP(32, TN, T, 0, 4, 4)         \
    FA_DECODE_LP(64, TN, T, 1, 4, 3)         \
    FA_DECODE_LP(64, TN, T, 0, 4, 3)         \
    FA_DECODE_LP(128, TN, T, 1, 3, 2)        \
    FA_DECODE_LP(128, TN, T, 0, 3, 2)        \
    FA_DECODE_LP(256, TN, T, 1, 1, 1)        \
    FA_DECODE_LP(256, TN, T, 0, 1, 1)
FA_DECODE_LP_ALL(bf16, __bf16)
FA_DECODE_LP_ALL(f16, _Float16)

// fa_decode_rows_d{D}_q{RQ}: row-streaming split-KV decode for seq_q <= RQ
// (f32, d % 4 == 0, 16-byte aligned operands).
#define FA_DECODE_ROWS(D, RQ)                                                                    \
    extern "C" __global__ void __launch_bounds__(256, 2) fa_decode_rows_d##D##_q##RQ(FaParams p) { \
        decode_rows_body<D, RQ>(p);                                                              \
    }
// fa_decode_rows_v1_d{D}_q{RQ}: the same with v1's per-block normalisation
#define FA_DECODE_ROWS_V1(D, RQ)                                                                 \
    extern "C" __global__ void __launch_bounds__(256, 2) fa_decode_rows_v1_d##D##_q##RQ(FaParams p) { \
        decode_rows_body<D, RQ, float, true>(p);                                                 \
    }
#define FA_DECODE_ROWS_ALL(D) FA_DECODE_ROWS(D, 1) FA_DECODE_ROWS(D, 2) FA_DECODE_ROWS(D, 4) \
    FA_DECODE_ROWS_V1(D, 1) FA_DECODE_ROWS_V1(D, 2) FA_DECODE_ROWS_V1(D, 4)
FA_DECODE_ROWS_ALL(32)
FA_DECODE_ROWS_ALL(64)
FA_DECODE_ROWS_ALL(128)
FA_DECODE_ROWS_ALL(256)
// fa_decode_rows_{bf16,f16}_d{D}_q1: 16-bit Q/K/V, seq_q = 1, d % 8 == 0,
// D >= 64 (more query rows would spill the widened chunks).
#define FA_DECODE_ROWS_LP(TN, T, D)                                                               \
    extern "C" __global__ void __launch_bounds__(256, 2) fa_decode_rows_##TN##_d##D##_q1(FaParams p) { \
        decode_rows_body<D, 1, T>(p);                                                            \
    }
#define FA_DECODE_ROWS_LP_ALL(TN, T) FA_DECODE_ROWS_LP(TN, T, 64) FA_DECODE_ROWS_LP(TN, T, 128) FA_DECODE_ROWS_LP(TN, T, 256)
FA_DECODE_ROWS_LP_ALL(bf16, __bf16)
FA_DECODE_ROWS_LP_ALL(f16, _Float16)

#define FA_MERGE(D) \
    extern "C" __global__ void __launch_bounds__(64 * FA_MERGE_ROWS) fa_merge_d##D(FaParams p) { merge_body<D>(p); }
// fa_merge_tiles_d{D}: the f32 prefill splits' merge (register-order tiles)
#define FA_MERGE_TILES(D) \
    extern "C" __global__ void __launch_bounds__(D) fa_merge_tiles_d##D(FaParams p) { merge_tiles_body<D>(p); }
FA_MERGE_TILES(64)
FA_MERGE_TILES(128)
FA_MERGE_TILES(256)
FA_MERGE(32)
FA_MERGE(64)
FA_MERGE(128)
FA_MERGE(256)
FA_MERGE(512)
FA_MERGE(1024)
FA_MERGE(2048)

#define FA_NAIVE(T, SUF)                                                                          \
    extern "C" __global__ void __launch_bounds__(256) fa_naive_scores_##SUF(NaiveParams p) {       \
        naive_scores_body<T>(p);                                                                  \
    }                                                                                             \
    extern "C" __global__ void __launch_bounds__(256) fa_naive_softmax_##SUF(NaiveParams p) {      \
        naive_softmax_body<T>(p);                                                                 \
    }                                                                                             \
    extern "C" __global__ void __launch_bounds__(256) fa_naive_pv_##SUF(NaiveParams p) { naive_pv_body<T>(p); }
FA_NAIVE(float, f32)
FA_NAIVE(double, f64)

#include "fa_lp.inc"

// ---------------------------------------------------------------------------
// Peak probes (new; no counterpart in the reference): the ceilings that the
// roofline fractions divide by, measured on the machine itself.
//  * fa_probe_mfma_*: every wave runs CH independent accumulator chains of
//    `iters` back-to-back MFMAs on lane-dependent inputs, then stores one
//    checksum; FLOP per launch = waves x iters x CH x FLOP per MFMA.  Each
//    chain's first step is peeled off the loop (from a zero accumulator): with
//    zero-initialised accumulators carried into it, the compiler shuffled
//    accumulator registers inside the loop (v_accvgpr_mov, 10 % of the rate).  A 64 KiB
//    LDS reservation holds the CU to two workgroups, two waves per SIMD as in
//    the attention kernels.
//  * fa_probe_copy: a grid-stride device copy of n16 16-byte elements from the
//    first half of the buffer to the second; bytes per launch = 2 x 16 x n16
//    (read + write).  (Measured: 5.7 TB/s; copies with each workgroup taking
//    one contiguous chunk, nontemporal or not, 5.2-5.3 TB/s.)
//  * fa_probe_read: a read-only stream of the buffer's first n16 16-byte
//    elements, each workgroup one contiguous chunk with sixteen nontemporal
//    1 KiB wave loads in flight (measured: 7.15 TB/s; grid-stride reads
//    5.1-5.5 TB/s); nothing is stored unless a lane's sum hits a value the
//    data never produces; bytes per launch = 16 x n16.
// ---------------------------------------------------------------------------
constexpr int kProbeLdsFloats = 16384;   // 64 KiB per workgroup

template <int KIND>
__device__ __forceinline__ void probe_mfma_body(const ProbeParams& p) {
    __shared__ float hold[kProbeLdsFloats];
    const int lane = threadIdx.x & 63;
    const unsigned wave = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    // the reservation is used, so it stays allocated
    hold[threadIdx.x * (kProbeLdsFloats / 256)] = (float)lane;
    __syncthreads();
    const float a = 1.0f + (float)lane * 1.0e-3f, b = 1.0f - (float)lane * 1.0e-3f;
    const unsigned iters = p.iters;
    float sum = 0.0f;
    if constexpr (KIND == 0) {
        constexpr int CH = 4;
        f32x16 acc[CH];
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) acc[ch] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, (f32x16){}, 0, 0, 0);
        for (unsigned it = 1; it < iters; ++it)
#pragma unroll
            for (int ch = 0; ch < CH; ++ch) acc[ch] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[ch], 0, 0, 0);
#pragma unroll
        for (int ch = 0; ch < CH; ++ch)
#pragma unroll
            for (int e = 0; e < 16; ++e) sum += acc[ch][e];
    } else if constexpr (KIND == 1) {
        constexpr int CH = 8;
        f32x4 acc[CH];
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) acc[ch] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, (f32x4){}, 0, 0, 0);
        for (unsigned it = 1; it < iters; ++it)
#pragma unroll
            for (int ch = 0; ch < CH; ++ch) acc[ch] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[ch], 0, 0, 0);
#pragma unroll
        for (int ch = 0; ch < CH; ++ch)
#pragma unroll
            for (int e = 0; e < 4; ++e) sum += acc[ch][e];
    } else {
        // KIND 2: v_mfma_f32_16x16x32_bf16, 16 chains; KIND 4: v_mfma_f32_32x32x16_bf16, 4 chains
        constexpr bool BIG = KIND == 4;
        constexpr int CH = BIG ? 4 : 16;
        typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
        bf16x8 va, vb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            va[e] = (__bf16)(a + (float)e * 1.0e-2f);
            vb[e] = (__bf16)(b - (float)e * 1.0e-2f);
        }
        typedef typename std::conditional<BIG, f32x16, f32x4>::type acc_t;
        constexpr int NE = BIG ? 16 : 4;
        acc_t acc[CH];
        auto step = [&](acc_t c) -> acc_t {
            if constexpr (BIG) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, vb, c, 0, 0, 0);
            else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, vb, c, 0, 0, 0);
        };
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) acc[ch] = step((acc_t){});
        for (unsigned it = 1; it < iters; ++it)
#pragma unroll
            for (int ch = 0; ch < CH; ++ch) acc[ch] = step(acc[ch]);
#pragma unroll
        for (int ch = 0; ch < CH; ++ch)
#pragma unroll
            for (int e = 0; e < NE; ++e) sum += acc[ch][e];
    }
    // read after the chains, so nothing but the accumulators is live across them
    sum += hold[(255 - threadIdx.x) * (kProbeLdsFloats / 256)] * 0.0f;
    if (lane == 0) p.buf[wave] = sum;
}

__device__ __forceinline__ void probe_copy_body(const ProbeParams& p) {
    const f32x4* __restrict__ src = reinterpret_cast<const f32x4*>(p.buf);
    f32x4* __restrict__ dst = reinterpret_cast<f32x4*>(p.buf) + p.n16;
    const unsigned long long n = p.n16;
    const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = src[i];
}

extern "C" __global__ void __launch_bounds__(256) fa_probe_mfma_f32_32x32x2(ProbeParams p) { probe_mfma_body<0>(p); }
extern "C" __global__ void __launch_bounds__(256) fa_probe_mfma_f32_16x16x4(ProbeParams p) { probe_mfma_body<1>(p); }
extern "C" __global__ void __launch_bounds__(256) fa_probe_mfma_bf16_16x16x32(ProbeParams p) { probe_mfma_body<2>(p); }
extern "C" __global__ void __launch_bounds__(256) fa_probe_copy(ProbeParams p) { probe_copy_body(p); }
extern "C" __global__ void __launch_bounds__(256) fa_probe_mfma_bf16_32x32x16(ProbeParams p) { probe_mfma_body<4>(p); }

__device__ __forceinline__ void probe_read_body(const ProbeParams& p) {
    constexpr int NF = 16;   // loads in flight per lane
    const f32x4* __restrict__ src = reinterpret_cast<const f32x4*>(p.buf);
    const unsigned long long n = p.n16, per = (n + gridDim.x - 1) / gridDim.x;
    const unsigned long long beg = (unsigned long long)blockIdx.x * per;
    const unsigned long long end = beg + per < n ? beg + per : n;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    unsigned long long i = beg + threadIdx.x;
    for (; i + (NF - 1) * 256 < end; i += NF * 256) {
        f32x4 x[NF];
#pragma unroll
        for (int j = 0; j < NF; ++j) x[j] = __builtin_nontemporal_load(src + i + j * 256);
#pragma unroll
        for (int j = 0; j < NF; ++j) acc += x[j];
    }
    for (; i < end; i += 256) acc += src[i];
    // keeps the loads; the buffer's contents never sum to this
    if (acc[0] == -1.0e30f) p.buf[blockIdx.x * blockDim.x + threadIdx.x] = acc[1];
}
extern "C" __global__ void __launch_bounds__(256) fa_probe_read(ProbeParams p) { probe_read_body(p); }
