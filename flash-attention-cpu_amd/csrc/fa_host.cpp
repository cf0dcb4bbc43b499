// fa_host.cpp -- host side of libfa_hip.so: the C ABI declared in
// include/fa_hip.h over the HIP runtime C API.
//
// Replaces the reference crate's entry / dispatch layer
// (amaye15/flash-attention-cpu): check_shapes (src/common.rs:41-57), the
// per-variant entry points (src/v1.rs:51-159, src/v2.rs:49-157,
// src/v3.rs:61-169) and multihead_dispatch (src/common.rs:72-101).  The
// crate's runtime ISA pick (src/v2.rs:63-120) becomes a pick among gfx950
// kernel instantiations (padded d_head, 128-bit vs scalar loads, prefill vs
// split-KV), and rayon's fan-out over (head, query block) becomes the
// launch grid.
//
// Kernels live in a code object (fa_kernels.hsaco, built from
// fa_kernels.hip) that is loaded once per device with hipModuleLoad and
// launched with hipModuleLaunchKernel.  There is no CPU compute path.

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/fa_hip.h"
#include "fa_copy_parts.h"
#include "fa_params.h"
#include "fa_scratch.h"

namespace {

constexpr int kMaxDevices = 64;
constexpr int kMaxD = 2048;         // widest head of the f32 flash kernels
constexpr int kMaxDNarrow = 256;    // 16-bit kernels and the split-KV decoders
constexpr int kDecodeRows = 16;     // query rows per split-KV wave
constexpr int kDecodeWaves = 4;     // waves per split-KV workgroup
constexpr int kRowsMaxQ = 4;        // row-streaming decode: most query rows

// Host-slice staging: pageable host memory moves through a ring of pinned
// buffers.  Host threads copy pageable <-> pinned while the DMA engine moves
// the previous buffer.  Measured on the MI355X box: pageable hipMemcpyAsync
// 25 GB/s host-to-device and 16 GB/s device-to-host; staged through 16 MiB
// pinned chunks with 4 host threads 54 GB/s both ways.
constexpr size_t kStageChunk = size_t(16) << 20;
constexpr int kStageBufs = 4;
constexpr int kCopyThreads = 4;     // host threads per staging copy, the caller included
constexpr size_t kCopySplitMin = size_t(1) << 20;   // smaller copies stay on the caller
// Transfers below this many bytes take plain pageable copies: the ring's
// per-chunk events cost more than they save on small calls (measured: a
// 256 x 64 single-head call 78 -> 111 us through the ring).
constexpr size_t kStageMinBytes = size_t(2) << 20;
// Host-slice calls in flight at once per device (each with its own stream,
// device staging buffer and pinned ring; further callers wait for one).
constexpr int kIoContexts = 4;

// One host-slice call's device-side resources: a stream, a grow-only device
// staging allocation and a ring of pinned buffers (allocated on first use).
struct IoContext {
    hipStream_t stream = nullptr;
    float* buf = nullptr;
    size_t floats = 0;
    char* pin = nullptr;              // kStageBufs x kStageChunk pinned bytes
    bool pin_tried = false;           // pinned ring unavailable: pageable copies
    hipEvent_t ev[kStageBufs] = {};   // last DMA on each ring buffer
};

struct DeviceState {
    std::once_flag once;
    int status = FA_OK;
    hipModule_t module = nullptr;
    int num_cus = 256;
    std::mutex fn_mu;
    std::unordered_map<std::string, hipFunction_t> fns;
    // Split workspaces (partials of split-KV / key split), one per stream,
    // grow-only: kernels on one stream run in order, so consecutive calls on
    // a stream can share one buffer, and calls on different streams never
    // share.  Saves the stream-ordered allocate / free per call (measured:
    // 5.5 us of idle GPU between back-to-back decode calls).
    struct Workspace {
        void* ptr = nullptr;
        size_t bytes = 0;
        std::vector<void*> retired;   // outgrown buffers: kept, a captured graph may name them
    };
    std::mutex ws_mu;
    std::unordered_map<std::string, Workspace> ws;   // freed by fa_release_stream_workspace
    // Host-slice calls: up to kIoContexts contexts, created as concurrent
    // callers need them and kept; a caller takes a free one for its call.
    std::mutex io_mu;
    std::condition_variable io_cv;
    std::vector<std::unique_ptr<IoContext>> io_all;
    std::vector<IoContext*> io_free;
};

// A small pool of host threads for large memcpy's.  One copy at a time
// (copy_mu); the caller takes the first part itself.
class CopyPool {
public:
    // Threads that cannot be started leave the pool smaller (with none, the
    // caller copies alone); no exception leaves the C ABI.
    explicit CopyPool(int workers) {
        try {
            for (int i = 0; i < workers; ++i) threads_.emplace_back([this, i] { work(i + 1); });
        } catch (...) {
        }
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> l(mu_);
            stop_ = true;
        }
        wake_.notify_all();
        for (auto& t : threads_) t.join();
    }
    void copy(void* dst, const void* src, size_t n) {
        if (threads_.empty() || n < kCopySplitMin) {
            std::memcpy(dst, src, n);
            return;
        }
        std::lock_guard<std::mutex> job(copy_mu_);
        const int parts = static_cast<int>(threads_.size()) + 1;
        {
            std::lock_guard<std::mutex> l(mu_);
            dst_ = static_cast<char*>(dst);
            src_ = static_cast<const char*>(src);
            n_ = n;
            parts_ = parts;
            pending_ = parts - 1;
            ++gen_;
        }
        wake_.notify_all();
        part(0, static_cast<char*>(dst), static_cast<const char*>(src), n, parts);
        std::unique_lock<std::mutex> l(mu_);
        done_.wait(l, [&] { return pending_ == 0; });
    }

private:
    static void part(int id, char* dst, const char* src, size_t n, int parts) {
        size_t b, len;
        fa_copy_part_range(n, parts, id, &b, &len);
        if (len) std::memcpy(dst + b, src + b, len);
    }
    void work(int id) {
        unsigned long seen = 0;
        std::unique_lock<std::mutex> l(mu_);
        for (;;) {
            wake_.wait(l, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            char* d = dst_;
            const char* s = src_;
            const size_t n = n_;
            const int parts = parts_;
            l.unlock();
            part(id, d, s, n, parts);
            l.lock();
            if (--pending_ == 0) done_.notify_one();
        }
    }
    std::vector<std::thread> threads_;
    std::mutex copy_mu_, mu_;
    std::condition_variable wake_, done_;
    unsigned long gen_ = 0;
    int pending_ = 0;
    bool stop_ = false;
    char* dst_ = nullptr;
    const char* src_ = nullptr;
    size_t n_ = 0;
    int parts_ = 1;
};

CopyPool& copy_pool() {
    static CopyPool pool(kCopyThreads - 1);
    return pool;
}

DeviceState g_dev[kMaxDevices];

std::string module_path() {
    const char* env = std::getenv("FA_HIP_MODULE");
    if (env && *env) return std::string(env);
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&fa_init), &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        const size_t pos = p.rfind('/');
        const std::string dir = (pos == std::string::npos) ? std::string(".") : p.substr(0, pos);
        return dir + "/fa_kernels.hsaco";
    }
    return "fa_kernels.hsaco";
}

int current_device(int* dev) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return FA_ERR_NO_DEVICE;
    }
    if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= kMaxDevices) return FA_ERR_NO_DEVICE;
    return FA_OK;
}

int ensure_loaded(int dev) {
    DeviceState& s = g_dev[dev];
    std::call_once(s.once, [&] {
        const std::string path = module_path();
        if (FILE* f = std::fopen(path.c_str(), "rb")) {
            std::fclose(f);
        } else {
            s.status = FA_ERR_MODULE;
            return;
        }
        if (hipModuleLoad(&s.module, path.c_str()) != hipSuccess) {
            (void)hipGetLastError();
            s.status = FA_ERR_MODULE;
            return;
        }
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
            s.num_cus = prop.multiProcessorCount;
        // Device address of the allocation-free entry point's scratch array;
        // a failure here concerns only that entry point (FA_ERR_SCRATCH).
        (void)fa_scratch_init(dev);
        s.status = FA_OK;
    });
    return s.status;
}

int get_function(int dev, const std::string& name, hipFunction_t* fn) {
    DeviceState& s = g_dev[dev];
    std::lock_guard<std::mutex> lock(s.fn_mu);
    auto it = s.fns.find(name);
    if (it != s.fns.end()) {
        *fn = it->second;
        return FA_OK;
    }
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, s.module, name.c_str()) != hipSuccess) {
        (void)hipGetLastError();
        return FA_ERR_MODULE;
    }
    s.fns.emplace(name, f);
    *fn = f;
    return FA_OK;
}

// ---------------------------------------------------------------------------
// Launch planning: which kernels, what grid, what workspace.
// ---------------------------------------------------------------------------
struct Launch {
    std::string name;
    unsigned gx = 1, gy = 1, gz = 1, bx = 1;
};

struct Plan {
    bool split = false;
    Launch first, second;   // second: the split-KV merge
    FaParams p{};
    size_t ws_floats = 0;   // split-KV workspace (part_o + part_ml)
};

// Most splits fa_merge's LDS weight table holds.
constexpr int kMaxSplits = 1024;
// Fewest keys per split-KV split the automatic plan makes.
constexpr size_t kMinSplitKeys = 256;

int pad_d(size_t d) {
    if (d <= 32) return 32;
    if (d <= 64) return 64;
    if (d <= 128) return 128;
    if (d <= 256) return 256;
    if (d <= 512) return 512;
    if (d <= 1024) return 1024;
    return 2048;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

int make_plan(int variant, const void* q, const void* k, const void* v, const float* out,
              size_t bh, size_t sq, size_t sk, size_t d, int causal, const fa_launch_opts* opts,
              int num_cus, Plan* plan) {
    if (variant < 1 || variant > 3) return FA_ERR_INVALID_ARG;
    const int path = opts ? opts->path : FA_PATH_AUTO;
    const int dtype = opts ? opts->dtype : FA_DTYPE_F32;
    if (dtype != FA_DTYPE_F32 && dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F16) return FA_ERR_INVALID_ARG;
    const bool lp = dtype != FA_DTYPE_F32;   // 16-bit inputs: the fa_prefill_lp kernels
    if (lp && variant == 1) return FA_ERR_INVALID_ARG;   // the 16-bit kernels run v2/v3's algorithm
    if (path < FA_PATH_AUTO || path > FA_PATH_STREAM) return FA_ERR_INVALID_ARG;
    if (opts && opts->num_splits < 0) return FA_ERR_INVALID_ARG;
    // d_head > 256: f32 prefill kernels only (column groups; key split allowed)
    const bool wide = d > (size_t)kMaxDNarrow;
    if (wide && (lp || path == FA_PATH_SPLITKV || path == FA_PATH_SPLITKV_ROWS)) return FA_ERR_UNSUPPORTED;
    // d_head > 2048: the any-width kernels only (one workgroup per 16-row
    // tile, no split of any kind)
    const bool any_width = d > (size_t)kMaxD;
    if (any_width && (path == FA_PATH_STREAM || (opts && opts->num_splits > 1))) return FA_ERR_UNSUPPORTED;
    const size_t imax = 0x7fffffff;
    if (sq > imax || sk > imax || bh > imax) return FA_ERR_UNSUPPORTED;

    const int D = pad_d(d);
    const bool vec = (d % (lp ? 8 : 4) == 0) && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
    float scale = 1.0f / std::sqrt(static_cast<float>(d));   // src/v2.rs:171
    if (opts && opts->softmax_scale > 0.0f && std::isfinite(opts->softmax_scale)) scale = opts->softmax_scale;

    FaParams& p = plan->p;
    std::memset(&p, 0, sizeof(p));
    p.q = static_cast<const float*>(q);   // 16-bit data for the lp kernels, which reinterpret
    p.k = static_cast<const float*>(k);
    p.v = static_cast<const float*>(v);
    p.out = const_cast<float*>(out);
    p.bh = static_cast<int>(bh);
    p.seq_q = static_cast<int>(sq);
    p.seq_k = static_cast<int>(sk);
    p.d = static_cast<int>(d);
    p.causal = causal ? 1 : 0;
    p.scale_log2e = scale * 1.44269504088896341f;
    // v1 visits every key of every query block (no causal skip,
    // src/v1.rs:209-216): its splits count each block's keys as all seq_k.
    p.full_keys = variant == 1 ? 1 : 0;
    const bool causal_skip = causal && variant != 1;

    if (any_width) {
        // O accumulates in `out` (no workspace); p.nqb counts 16-row tiles
        const size_t tiles = (sq + 15) / 16;
        if (tiles * bh > imax || d > imax) return FA_ERR_UNSUPPORTED;
        const bool vec_any = d % 4 == 0 && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
        char nm[64];
        // up to 4096 columns (8 waves x 8 chunks of 64) each wave keeps its
        // chunks of O in registers; wider heads accumulate in `out`
        std::snprintf(nm, sizeof(nm), "fa_prefill_v%d_%s_%d", variant, d <= 4096 ? "dreg" : "dany", vec_any ? 1 : 0);
        plan->first.name = nm;
        plan->first.gx = static_cast<unsigned>(tiles * bh);
        plan->first.bx = 512;
        p.nqb = static_cast<int>(tiles);
        plan->split = false;
        plan->ws_floats = 0;
        return FA_OK;
    }

    const size_t rows = (size_t)(lp ? fa_lp_rows() : fa_prefill_rows(D));   // query rows per prefill workgroup
    const size_t nqb = (sq + rows - 1) / rows;
    const size_t nqt = (sq + kDecodeRows - 1) / kDecodeRows;
    // Row-streaming decode: 16-byte loads; f32 with seq_q <= 4, or 16-bit
    // with seq_q = 1 and D >= 64.
    const bool rows_ok = !wide && vec && (lp ? (sq == 1 && D >= 64) : sq <= (size_t)kRowsMaxQ);
    if (path == FA_PATH_SPLITKV_ROWS && !rows_ok) return FA_ERR_UNSUPPORTED;
    // Decode steps (at most two 16-row tiles) take split-KV whatever the
    // grid and the key count: a prefill block would hold 1-32 valid rows of
    // 128 and stream K / V through LDS at under 2 TB/s (measured on MI355X,
    // d128: 512 slices x 1 query x 1024 keys 285 -> 77 us, 256 x 32 x 2048
    // 283 -> 162 us, 512 x 1 x 64 21.2 -> 5.5 us, 256 x 16 x 64 11.4 -> 7.7
    // us; at 64 queries and 256 slices the tiles' four K / V passes cost
    // more, 639 against 558 us).  16-bit inputs: the row kernel only (sq =
    // 1: 14.6 -> 12.7 us at 256 keys, 44.1 -> 42.1 at 1024; 16 rows stay on
    // the 16-bit prefill, 45.9 against 104.7 us).
    const bool step_shape = sq <= 2 * (size_t)kDecodeRows && (!lp || rows_ok);
    bool split = false;
    {   // every variant: v1's split kernels keep its per-block normalisation
        if (path == FA_PATH_SPLITKV || path == FA_PATH_SPLITKV_ROWS) {
            split = true;
        } else if (path == FA_PATH_AUTO && !wide && step_shape) {
            split = true;
        } else if (path == FA_PATH_AUTO && nqb * bh < (size_t)num_cus) {
            // Grids smaller than the GPU.  Decode shapes take split-KV.  So do
            // small f32 prefills: at most num_cus/2 16-row tiles and 256 keys
            // or more, where 16-row tiles x key splits occupy the GPU better
            // than the key-split prefill (measured on MI355X: 2.0-3.8x faster
            // up to 128 tiles x heads, e.g. config 1 20.6 -> 8.2 us; 0.5-0.8x
            // from 188 on, where re-reading K / V per tile costs more).
            // 16-bit inputs: the key-split 16-bit prefill is faster than the
            // 16-row widening split-KV kernel (113 vs 148 us on config 4), so
            // they take split-KV only where the row kernel applies.
            const bool decode_shape = sq <= 64 && sk >= 512;
            const bool few_tiles = !lp && nqt * bh * 2 <= (size_t)num_cus && sk >= 256;
            split = !wide && (decode_shape || few_tiles) && (!lp || rows_ok);
        }
    }
    const bool row_decode = split && rows_ok && (path == FA_PATH_SPLITKV_ROWS || path == FA_PATH_AUTO);
    // split-KV grid: splits x tiles x slices workgroups in one dimension
    if (split && nqt * bh > imax / (size_t)kMaxSplits) {
        if (path == FA_PATH_SPLITKV || path == FA_PATH_SPLITKV_ROWS) return FA_ERR_UNSUPPORTED;
        split = false;
    }
    plan->split = split;
    char buf[64];
    if (!split) {
        if (nqb * bh > imax) return FA_ERR_UNSUPPORTED;
        p.nqb = static_cast<int>(nqb);
        int lp_tiles = 1;
        // 16-bit stream split (forced only): the two-tile kernel at D = 128.
        // AUTO does not take it: measured on config 2 causal bf16 (46.9 ->
        // 89.9 us) and config 3 (489 -> 568 us), the partials of the split
        // blocks and their merge cost more than the even runs save at
        // 16-bit speed.
        const bool lp_stream = lp && D == 128 && variant != 1 && path == FA_PATH_STREAM;
        if (lp) {
            // Two 16-row tiles per wave halve LDS traffic per row but leave one
            // wave per SIMD in a workgroup running alone: worth it at D = 128
            // unless the grid is a single round of unequal causal blocks (the
            // stream split evens those out).
            if (D == 128 && (lp_stream || !causal || nqb * bh > 2 * (size_t)num_cus)) lp_tiles = 2;
            // 0: register-staged scalar loads (any d), 2: global->LDS DMA
            std::snprintf(buf, sizeof(buf), "fa_prefill_lp_%s_d%d_%d_t%d", dtype == FA_DTYPE_BF16 ? "bf16" : "f16",
                          D, vec ? 2 : 0, lp_tiles);
        } else {
            // 0: scalar loads (any d), 1: 128-bit loads, 2: global->LDS DMA (v3:
            // two LDS stages, or at D = 1024 alternating K and V buffers; not
            // at D = 2048)
            const int loader = vec ? (fa_prefill_dma(D, variant) ? 2 : 1) : 0;
            std::snprintf(buf, sizeof(buf), "fa_prefill_v%d_d%d_%d", variant, D, loader);
        }
        plan->first.name = buf;
        plan->first.gx = static_cast<unsigned>(nqb * bh);
        plan->first.bx = 64 * (lp ? fa_lp_waves(lp_tiles) : fa_prefill_waves(D));
        // The 16-bit kernels fit two workgroups per CU for D <= 128.
        if (lp && D <= 128 && causal && bh <= (size_t)num_cus && num_cus % bh == 0)
            p.pair_w = static_cast<int>(num_cus / bh);
        plan->ws_floats = 0;
        // Key split for v2/v3 when the grid would leave CUs idle: a query
        // block's keys are cut into splits of `per` stages, one workgroup
        // each (the split instantiation, name suffix "s"), whose partials
        // fa_merge combines.  Causal blocks differ in
        // length, so `per` is chosen to minimise the estimated makespan in
        // key-steps: rounds of resident workgroups (one per CU) x (keys per
        // split + kOverheadKeys for loading Q and writing the partial), plus
        // kOverheadKeys per round for the merge's re-read; at least four
        // stages per split.  Measured on MI355X, a single round of long
        // splits beats several rounds of short ones.  The grid lists only
        // workgroups with keys.
        size_t per = 0;
        // The prefill splits' merge: the f32 split kernels at D = 64, 128,
        // 256 write their partial tiles in register order, merged a
        // workgroup per 16-row tile (a wave per 64 columns); the others
        // (D = 32, column groups, 16-bit) by rows, a wave per row.
        auto prefill_merge = [&]() {
            if (!lp && (D == 64 || D == 128 || D == 256)) {
                std::snprintf(buf, sizeof(buf), "fa_merge_tiles_d%d", D);
                plan->second.gx = static_cast<unsigned>(nqt * bh);
                plan->second.bx = static_cast<unsigned>(D);
            } else {
                std::snprintf(buf, sizeof(buf), "fa_merge_d%d", D);
                plan->second.gx = static_cast<unsigned>((bh * sq + FA_MERGE_ROWS - 1) / FA_MERGE_ROWS);   // a wave per row
                plan->second.bx = 64 * FA_MERGE_ROWS;
            }
            plan->second.name = buf;
        };
        {
            const size_t SKs = (size_t)(lp ? fa_lp_stage_keys() : fa_prefill_stage_keys(D, variant));
            auto block_stages = [&](size_t b) {
                const size_t kend = causal_skip ? std::min(sk, (b + 1) * rows) : sk;
                return (kend + SKs - 1) / SKs;
            };
            const size_t max_st = block_stages(nqb - 1);   // causal key ends grow with the block
            auto wgs_for = [&](size_t pp) {
                size_t n = 0;
                for (size_t b = 0; b < nqb; ++b) n += (block_stages(b) + pp - 1) / pp;
                return n * bh;
            };
            constexpr double kOverheadKeys = 48.0;
            // Stream split (f32 v2/v3): the key stages of all (slice, query
            // block) pairs, slice-major, cut into equal runs of s_per stages,
            // one run per workgroup (want of them); a block shared by several
            // runs is merged from one partial per run, kept in block slot
            // (workgroup + global block index): workgroups + blocks - 1
            // slots of `rows` rows.  Block b has
            // R (b + 1) stages while (b + 1) * rows <= seq_k (causal), else
            // ceil(seq_k / SK); rows is a multiple of SK.
            size_t s_per = 0, s_wgs = 0, s_segs = 0, s_uhead = 0;
            auto stream_fit = [&](size_t want) -> bool {
                const size_t R = rows / SKs, nsf = (sk + SKs - 1) / SKs, bf = sk / rows;
                const size_t b = nqb;
                s_uhead = !causal_skip ? b * nsf
                                       : (b <= bf ? R * (b * (b + 1) / 2) : R * (bf * (bf + 1) / 2) + (b - bf) * nsf);
                // The kernel keeps unit indices (up to the total plus one
                // run) in 32 bits: larger totals are refused (AUTO then keeps
                // the key split; a forced stream split is unsupported).
                if (s_uhead == 0 || s_uhead > imax || bh > imax / s_uhead) return false;
                const size_t utot = bh * s_uhead;
                s_per = std::max<size_t>(4, (utot + want - 1) / want);
                s_wgs = (utot + s_per - 1) / s_per;
                s_segs = (max_st + s_per - 1) / s_per + 1;   // most workgroups sharing a block
                return s_segs <= (size_t)kMaxSplits && utot + s_per <= imax && s_wgs <= imax && bh * sq <= imax &&
                       s_wgs + bh * nqb <= imax;
            };
            // workgroups resident at once: the 16-bit kernels fit two per CU at D <= 128
            const size_t resident = (size_t)num_cus * (lp && D <= 128 ? 2 : 1);
            bool stream = false;
            if (path == FA_PATH_STREAM) {
                if (opts->num_splits > 0 && (size_t)opts->num_splits > imax) return FA_ERR_UNSUPPORTED;
                if (!stream_fit(opts->num_splits > 0 ? (size_t)opts->num_splits : resident)) return FA_ERR_UNSUPPORTED;
                stream = true;
            } else if (opts && opts->num_splits > 1 && path == FA_PATH_PREFILL) {
                if (opts->num_splits > kMaxSplits) return FA_ERR_UNSUPPORTED;
                per = (max_st + opts->num_splits - 1) / opts->num_splits;
            } else if (path == FA_PATH_AUTO && nqb * bh < (size_t)num_cus) {
                const double cus = (double)num_cus, skd = (double)SKs;
                double best = std::ceil((double)(nqb * bh) / cus) * (double)max_st * skd;   // no split
                // Candidates: for R = 1..4 rounds, the shortest split whose
                // workgroups fit in R rounds (workgroup count falls as `per`
                // grows, so bisect).
                for (size_t R = 1; R <= 4; ++R) {
                    const size_t slots = R * (size_t)num_cus;
                    size_t lo = 4, hi = max_st;
                    if (lo > hi || wgs_for(hi) > slots) continue;
                    while (lo < hi) {
                        const size_t mid = (lo + hi) / 2;
                        if (wgs_for(mid) <= slots) hi = mid;
                        else lo = mid + 1;
                    }
                    const size_t pp = lo;
                    const double n = (double)wgs_for(pp);
                    const double cost = std::ceil(n / cus) * ((double)pp * skd + kOverheadKeys) + n / cus * kOverheadKeys;
                    if (cost < best) {
                        best = cost;
                        per = pp;
                    }
                }
                // The stream split: one round, up to two segment prologues
                // per workgroup and the merge of the shared blocks.
                if (!lp && stream_fit((size_t)num_cus)) {
                    const double cost = (double)s_per * skd + 3.0 * kOverheadKeys;
                    if (cost < best) {
                        best = cost;
                        per = 0;
                        stream = true;
                    }
                }
            }
            if (stream) {
                plan->first.name += "s";   // the stream-split instantiation
                plan->split = true;
                p.nqt = static_cast<int>(nqt);
                p.num_splits = static_cast<int>(s_segs);
                p.split_len = static_cast<int>(SKs);
                p.ks_rows = static_cast<int>(rows);
                p.merge_scale = 1.0f;
                p.pair_w = 0;
                p.stream_per = static_cast<long long>(s_per);
                p.stream_head_units = static_cast<long long>(s_uhead);
                plan->first.gx = static_cast<unsigned>(s_wgs);
                prefill_merge();
                plan->ws_floats = (s_wgs + bh * nqb - 1) * (rows / 16) * (16 * (size_t)D + 32);
                return FA_OK;
            }
            if (per > 0 && (max_st + per - 1) / per < 2) per = 0;
            if (per > 0 && (bh * sq > imax || per * SKs > imax)) return FA_ERR_UNSUPPORTED;
            // f32 v3 with 128-bit DMA and d = D = 128: pair query blocks nqb-1-r
            // and r in one workgroup (equal causal work per workgroup; the
            // second block's loads overlap the first's last step) when the
            // pairs fill whole rounds of one workgroup per CU.
            if (per == 0 && !lp && variant == 3 && vec && (size_t)D == d && D == 128 && nqb % 2 == 0 &&
                (nqb / 2 * bh) % (size_t)num_cus == 0) {
                p.two_blocks = 1;
                plan->first.gx = static_cast<unsigned>(nqb / 2 * bh);
            }
            if (per > 0) {
                const size_t nks = (max_st + per - 1) / per;
                if (nks > 65535 || nks > (size_t)kMaxSplits) return FA_ERR_UNSUPPORTED;
                plan->first.name += "s";   // the split instantiation
                plan->split = true;
                p.nqt = static_cast<int>(nqt);
                p.num_splits = static_cast<int>(nks);
                p.split_len = static_cast<int>(per * SKs);
                p.ks_rows = static_cast<int>(rows);
                p.merge_scale = 1.0f;   // prefill partial maxima are in the log2 domain
                p.pair_w = 0;           // the compact split grid has its own order
                size_t wgs = 0;   // compact grid: split y of every block that reaches it
                for (size_t y = 0; y < nks; ++y)
                    wgs += (causal_skip ? nqb - std::min(nqb, y * per * SKs / rows) : nqb) * bh;
                if (wgs > imax) return FA_ERR_UNSUPPORTED;
                plan->first.gx = static_cast<unsigned>(wgs);
                prefill_merge();
                plan->ws_floats = bh * nqt * nks * (16 * (size_t)D + 32);
            }
        }
        return FA_OK;
    }
    // Split-KV: each workgroup takes split_len keys (a multiple of 64) for one
    // (bh, 16-row query tile).  By default the split count fills exactly one
    // round of resident workgroups (no tail), with at least 64 keys each.
    size_t nsplit;
    if (opts && opts->num_splits > 0) {
        nsplit = (size_t)opts->num_splits;
    } else {
        // Workgroups to fill the GPU: the row-streaming kernel and the
        // 16-row tiles of small prefills two per CU (D = 256 tiles: one,
        // with 424 of 512 registers per lane); the tiles of decode steps one
        // per CU with longer splits (measured on MI355X, d128: 64 x 16 x
        // 4096 4 splits 47.0 us against 8 splits 51.3, config 4b 164.0
        // against 168.1; while causal 1 x 2048^2 takes 29.0 us in 4 splits
        // against 31.8 in 2).  At least kMinSplitKeys keys per split:
        // shorter ones cost more in per-workgroup set-up and merge than they
        // gain (1 x 1 x 8192: 32 splits 8.2 us, 128 splits 9.2; config 1 in
        // one split, no merge: 6.4 against 7.4 us).
        const size_t wg_per_cu = row_decode ? 2 : (D <= 128 && !step_shape ? 2 : 1);
        const size_t slots = wg_per_cu * (size_t)num_cus;
        nsplit = slots / (nqt * bh);
        if (nsplit < 1) nsplit = 1;
        if (nsplit > (size_t)kMaxSplits) nsplit = kMaxSplits;
        nsplit = std::min(nsplit, std::max<size_t>(1, sk / kMinSplitKeys));
    }
    size_t split_len = (sk + nsplit - 1) / nsplit;
    split_len = ((split_len + 63) / 64) * 64;
    nsplit = (sk + split_len - 1) / split_len;
    if (nsplit > (size_t)kMaxSplits || split_len > imax) return FA_ERR_UNSUPPORTED;
    p.nqt = static_cast<int>(nqt);
    p.num_splits = static_cast<int>(nsplit);
    p.split_len = static_cast<int>(split_len);
    p.merge_scale = p.scale_log2e;   // decode partial maxima are raw scores
    // v1: the instantiations with its per-block normalisation ("_v1")
    const char* v1tag = variant == 1 ? "v1_" : "";
    if (row_decode) {
        const int rq = sq <= 1 ? 1 : (sq <= 2 ? 2 : 4);
        if (lp)
            std::snprintf(buf, sizeof(buf), "fa_decode_rows_%s_d%d_q1", dtype == FA_DTYPE_BF16 ? "bf16" : "f16", D);
        else
            std::snprintf(buf, sizeof(buf), "fa_decode_rows_%sd%d_q%d", v1tag, D, rq);
    } else if (lp) {
        // 16-bit K/V streamed and widened in registers: 8-byte loads need d % 4 == 0
        const bool vec8 = (d % 4 == 0) && aligned8(q) && aligned8(k) && aligned8(v) && aligned16(out);
        std::snprintf(buf, sizeof(buf), "fa_decode_%s_d%d_%d", dtype == FA_DTYPE_BF16 ? "bf16" : "f16", D,
                      vec8 ? 1 : 0);
    } else {
        // 0: scalar loads, 1: 16-byte loads, 2: K through per-wave LDS rings (D = 64, 128)
        std::snprintf(buf, sizeof(buf), "fa_decode_%sd%d_%d", v1tag, D, vec ? (D == 64 || D == 128 ? 2 : 1) : 0);
    }
    plan->first.name = buf;
    plan->first.gx = static_cast<unsigned>(nsplit * nqt * bh);   // split-fastest, then tile, then slice
    plan->first.bx = 64 * kDecodeWaves;
    if (nsplit == 1) {
        // one split: each workgroup sees all keys of its rows and writes
        // them normalised (no partials, no merge)
        plan->split = false;
        plan->ws_floats = 0;
        return FA_OK;
    }
    std::snprintf(buf, sizeof(buf), "fa_merge_d%d", D);
    plan->second.name = buf;
    plan->second.gx = static_cast<unsigned>((bh * sq + FA_MERGE_ROWS - 1) / FA_MERGE_ROWS);   // a wave per row
    plan->second.bx = 64 * FA_MERGE_ROWS;
    plan->ws_floats = bh * nqt * nsplit * (16 * (size_t)D + 32);
    return FA_OK;
}

int launch(int dev, const Launch& L, FaParams* p, hipStream_t stream) {
    hipFunction_t fn;
    int rc = get_function(dev, L.name, &fn);
    if (rc != FA_OK) return rc;
    void* args[] = {p};
    if (hipModuleLaunchKernel(fn, L.gx, L.gy, L.gz, L.bx, 1, 1, 0, stream, args, nullptr) != hipSuccess) {
        (void)hipGetLastError();
        return FA_ERR_LAUNCH;
    }
    return FA_OK;
}

// Largest split workspace kept per stream; larger ones are allocated and
// released stream-ordered around the call.
constexpr size_t kWorkspaceCacheMax = size_t(256) << 20;

// The split workspace of `stream` on `dev`, at least `bytes` long.  Grows
// geometrically with hipMalloc (not a stream operation, so a first call under
// graph capture does not turn the buffer into graph-owned memory); an
// outgrown buffer is kept, not freed, since work already queued on the stream
// -- or a graph captured earlier -- may still use it.  hipStreamPerThread
// names a different stream in every thread, so its key includes the thread.
std::string workspace_key(hipStream_t stream) {
    char key[64];
    if (stream == hipStreamPerThread) {
        const size_t tid = std::hash<std::thread::id>{}(std::this_thread::get_id());
        std::snprintf(key, sizeof(key), "pt:%zx", tid);
    } else {
        std::snprintf(key, sizeof(key), "%p", reinterpret_cast<void*>(stream));
    }
    return key;
}

// Device memory free right now (0 when the query fails).
size_t free_device_bytes() {
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return free_b;
}

//
// A call captured into a graph takes the buffer over: it moves to the
// stream's retired list (kept until fa_release_stream_workspace), and the
// next eager call on the stream gets a new one.  So replays of the graph --
// on any stream -- never share partials with later eager calls on the
// capture stream, nor with another graph captured there.
int stream_workspace(int dev, hipStream_t stream, size_t bytes, void** out) {
    DeviceState& s = g_dev[dev];
    const std::string key = workspace_key(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) {
        (void)hipGetLastError();
        cap = hipStreamCaptureStatusNone;
    }
    const bool capturing = cap == hipStreamCaptureStatusActive;
    std::lock_guard<std::mutex> lock(s.ws_mu);
    DeviceState::Workspace& w = s.ws[key];
    if (capturing) {
        void* ptr = nullptr;
        if (w.ptr && w.bytes >= bytes) {
            ptr = w.ptr;
            w.ptr = nullptr;
            w.bytes = 0;
        } else if (hipMalloc(&ptr, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return FA_ERR_ALLOC;
        }
        w.retired.push_back(ptr);
        *out = ptr;
        return FA_OK;
    }
    if (w.ptr && w.bytes >= bytes) {
        *out = w.ptr;
        return FA_OK;
    }
    const size_t want = std::max({bytes, 2 * w.bytes, size_t(1) << 20});
    void* ptr = nullptr;
    if (hipMalloc(&ptr, want) != hipSuccess) {
        (void)hipGetLastError();
        return FA_ERR_ALLOC;
    }
    if (w.ptr) w.retired.push_back(w.ptr);
    w.ptr = ptr;
    w.bytes = want;
    *out = ptr;
    return FA_OK;
}

// Queue one attention call on device pointers.  noalloc: the split
// partials go to the device-global scratch array (fa_scratch.hip) and the
// call allocates nothing; plans needing more than it holds are refused.
int run_device(int variant, hipStream_t stream, const void* q, const void* k, const void* v, size_t bh,
               size_t sq, size_t sk, size_t d, int causal, const fa_launch_opts* opts, float* out,
               bool noalloc = false) {
    if (bh == 0 || sq == 0 || sk == 0 || d == 0) return FA_OK;   // src/common.rs:56
    if (!q || !k || !v || !out) return FA_ERR_INVALID_ARG;
    int dev;
    int rc = current_device(&dev);
    if (rc != FA_OK) return rc;
    rc = ensure_loaded(dev);
    if (rc != FA_OK) return rc;
    Plan plan;
    rc = make_plan(variant, q, k, v, out, bh, sq, sk, d, causal, opts, g_dev[dev].num_cus, &plan);
    if (rc != FA_OK) return rc;
    if (!plan.split) return launch(dev, plan.first, &plan.p, stream);

    const size_t bytes = plan.ws_floats * sizeof(float);
    float* ws = nullptr;
    const bool cached = noalloc || bytes <= kWorkspaceCacheMax;
    if (noalloc) {
        ws = static_cast<float*>(fa_scratch_ptr(dev));
        if (!ws || bytes > FA_SCRATCH_BYTES) return FA_ERR_SCRATCH;
    } else if (cached) {
        rc = stream_workspace(dev, stream, bytes, reinterpret_cast<void**>(&ws));
        if (rc != FA_OK) return rc;
    } else if (bytes > free_device_bytes() ||
               hipMallocAsync(reinterpret_cast<void**>(&ws), bytes, stream) != hipSuccess) {
        (void)hipGetLastError();
        return FA_ERR_ALLOC;   // nothing queued, out untouched
    }
    const int D = pad_d(d);
    const size_t parts = plan.ws_floats / (16 * (size_t)D + 32);   // 16-row partials: O, then (m, l)
    plan.p.part_o = ws;
    plan.p.part_ml = ws + parts * 16 * D;
    rc = launch(dev, plan.first, &plan.p, stream);
    if (rc == FA_OK) rc = launch(dev, plan.second, &plan.p, stream);
    if (!cached && hipFreeAsync(ws, stream) != hipSuccess) {
        (void)hipGetLastError();
        if (rc == FA_OK) rc = FA_ERR_ALLOC;
    }
    return rc;
}

int check_single(size_t q_len, size_t k_len, size_t v_len, size_t out_len, size_t sq, size_t sk,
                 size_t d) {
    if (q_len != sq * d) return FA_ERR_Q_SHAPE;
    if (k_len != sk * d) return FA_ERR_K_SHAPE;
    if (v_len != sk * d) return FA_ERR_V_SHAPE;
    if (out_len != sq * d) return FA_ERR_OUT_SHAPE;
    return FA_OK;
}

// The pinned ring of `s` (allocated on first use; false when pinned memory
// is unavailable, and host slices then take pageable copies).
bool stage_ring(IoContext& s) {
    if (s.pin) return true;
    if (s.pin_tried) return false;
    s.pin_tried = true;
    void* pin = nullptr;
    if (hipHostMalloc(&pin, kStageBufs * kStageChunk, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    for (int b = 0; b < kStageBufs; ++b) {
        if (hipEventCreateWithFlags(&s.ev[b], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            for (int c = 0; c < b; ++c) (void)hipEventDestroy(s.ev[c]);
            (void)hipHostFree(pin);
            return false;
        }
    }
    s.pin = static_cast<char*>(pin);
    return true;
}

struct HostSeg {
    char* dev;
    const char* host;
    size_t bytes;
};

// Host -> device through the pinned ring: each chunk is copied into a ring
// buffer by the copy pool, then queued as a DMA on `st`; a buffer is refilled
// once its previous DMA has completed.
int stage_up(IoContext& s, hipStream_t st, const HostSeg* segs, int nseg) {
    int slot = 0;
    bool used[kStageBufs] = {};
    for (int i = 0; i < nseg; ++i) {
        for (size_t off = 0; off < segs[i].bytes; off += kStageChunk) {
            const size_t len = std::min(kStageChunk, segs[i].bytes - off);
            char* buf = s.pin + slot * kStageChunk;
            if (used[slot] && hipEventSynchronize(s.ev[slot]) != hipSuccess) return FA_ERR_COPY;
            copy_pool().copy(buf, segs[i].host + off, len);
            if (hipMemcpyAsync(segs[i].dev + off, buf, len, hipMemcpyHostToDevice, st) != hipSuccess ||
                hipEventRecord(s.ev[slot], st) != hipSuccess)
                return FA_ERR_COPY;
            used[slot] = true;
            slot = (slot + 1) % kStageBufs;
        }
    }
    return FA_OK;
}

// Device -> host through the pinned ring: up to kStageBufs chunks in flight;
// each is copied out by the copy pool when its DMA has completed.
int stage_down(IoContext& s, hipStream_t st, char* host, const char* dev, size_t bytes) {
    const size_t nch = (bytes + kStageChunk - 1) / kStageChunk;
    auto queue = [&](size_t c) {
        const size_t off = c * kStageChunk, len = std::min(kStageChunk, bytes - off);
        const int b = static_cast<int>(c % kStageBufs);
        return hipMemcpyAsync(s.pin + b * kStageChunk, dev + off, len, hipMemcpyDeviceToHost, st) ==
                       hipSuccess &&
               hipEventRecord(s.ev[b], st) == hipSuccess;
    };
    for (size_t c = 0; c < nch && c < (size_t)kStageBufs; ++c)
        if (!queue(c)) return FA_ERR_COPY;
    for (size_t c = 0; c < nch; ++c) {
        const int b = static_cast<int>(c % kStageBufs);
        const size_t off = c * kStageChunk, len = std::min(kStageChunk, bytes - off);
        if (hipEventSynchronize(s.ev[b]) != hipSuccess) return FA_ERR_COPY;
        copy_pool().copy(host + off, s.pin + b * kStageChunk, len);
        if (c + kStageBufs < nch && !queue(c + kStageBufs)) return FA_ERR_COPY;
    }
    return FA_OK;
}

// A free host-slice context of device `dev` for the duration of one call:
// an idle one, a new one while fewer than kIoContexts exist, or the next one
// another caller releases.  Its stream is created with the context.
class IoLease {
public:
    explicit IoLease(DeviceState& s) : s_(s) {
        std::unique_lock<std::mutex> l(s_.io_mu);
        s_.io_cv.wait(l, [&] { return !s_.io_free.empty() || s_.io_all.size() < (size_t)kIoContexts; });
        if (!s_.io_free.empty()) {
            ctx_ = s_.io_free.back();
            s_.io_free.pop_back();
            return;
        }
        std::unique_ptr<IoContext> c(new (std::nothrow) IoContext());
        if (!c) return;
        if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
            (void)hipGetLastError();
            return;
        }
        ctx_ = c.get();
        s_.io_all.push_back(std::move(c));
    }
    ~IoLease() {
        if (!ctx_) return;
        {
            std::lock_guard<std::mutex> l(s_.io_mu);
            s_.io_free.push_back(ctx_);
        }
        s_.io_cv.notify_one();
    }
    IoContext* get() const { return ctx_; }

private:
    DeviceState& s_;
    IoContext* ctx_ = nullptr;
};

// Host slices: copy in (Q/K/V elements of `esize` bytes), run
// `run(stream, dq, dk, dv, dout)` on the device copies, copy the f32 output
// out, synchronise.  Up to kIoContexts calls per device run at once, each on
// its own context (the reference's functions are Sync and run concurrently
// from several threads: src/v2.rs:49-157).
template <typename F>
int with_host_slices(const void* q, const void* k, const void* v, size_t esize, size_t bh, size_t sq, size_t sk,
                     size_t d, float* out, F&& run) {
    int dev;
    int rc = current_device(&dev);
    if (rc != FA_OK) return rc;
    rc = ensure_loaded(dev);
    if (rc != FA_OK) return rc;
    IoLease lease(g_dev[dev]);
    if (!lease.get()) return FA_ERR_LAUNCH;
    IoContext& s = *lease.get();
    // Regions rounded up to 256 bytes keep every operand 256-byte aligned.
    auto up = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const size_t nq = bh * sq * d, nk = bh * sk * d;
    const size_t bq = up(nq * esize), bk = up(nk * esize), bo = up(nq * sizeof(float));
    const size_t need = (bq + 2 * bk + bo + sizeof(float) - 1) / sizeof(float);
    if (need > s.floats) {
        if (s.buf) (void)hipFree(s.buf);
        s.buf = nullptr;
        s.floats = 0;
        if (hipMalloc(reinterpret_cast<void**>(&s.buf), need * sizeof(float)) != hipSuccess) {
            (void)hipGetLastError();
            return FA_ERR_ALLOC;
        }
        s.floats = need;
    }
    char* base = reinterpret_cast<char*>(s.buf);
    void* dq = base;
    void* dk = base + bq;
    void* dv = base + bq + bk;
    float* dout = reinterpret_cast<float*>(base + bq + 2 * bk);
    hipStream_t st = s.stream;
    // On an error, queued DMA may still use the ring: drain the stream first.
    auto fail = [&](int code) {
        (void)hipGetLastError();
        (void)hipStreamSynchronize(st);
        (void)hipGetLastError();
        return code;
    };
    const bool staged_up = (nq + 2 * nk) * esize >= kStageMinBytes && stage_ring(s);
    const bool staged_down = nq * sizeof(float) >= kStageMinBytes && stage_ring(s);
    if (staged_up) {
        const HostSeg segs[3] = {{static_cast<char*>(dq), static_cast<const char*>(q), nq * esize},
                                 {static_cast<char*>(dk), static_cast<const char*>(k), nk * esize},
                                 {static_cast<char*>(dv), static_cast<const char*>(v), nk * esize}};
        if (stage_up(s, st, segs, 3) != FA_OK) return fail(FA_ERR_COPY);
    } else if (hipMemcpyAsync(dq, q, nq * esize, hipMemcpyHostToDevice, st) != hipSuccess ||
               (nk > 0 && hipMemcpyAsync(dk, k, nk * esize, hipMemcpyHostToDevice, st) != hipSuccess) ||
               (nk > 0 && hipMemcpyAsync(dv, v, nk * esize, hipMemcpyHostToDevice, st) != hipSuccess)) {
        return fail(FA_ERR_COPY);
    }
    rc = run(st, dq, dk, dv, dout);
    if (rc != FA_OK) return fail(rc);
    if (staged_down) {
        if (stage_down(s, st, reinterpret_cast<char*>(out), reinterpret_cast<const char*>(dout),
                       nq * sizeof(float)) != FA_OK)
            return fail(FA_ERR_COPY);
    } else if (hipMemcpyAsync(out, dout, nq * sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess) {
        return fail(FA_ERR_COPY);
    }
    if (hipStreamSynchronize(st) != hipSuccess) return fail(FA_ERR_COPY);
    return FA_OK;
}

int run_host(int variant, const float* q, const float* k, const float* v, size_t bh, size_t sq, size_t sk,
             size_t d, const fa_config* cfg, float* out) {
    if (bh == 0 || sq == 0 || sk == 0 || d == 0) return FA_OK;   // out untouched
    if (!q || !k || !v || !out) return FA_ERR_INVALID_ARG;
    const int causal = cfg ? cfg->causal : 0;
    return with_host_slices(q, k, v, sizeof(float), bh, sq, sk, d, out,
                            [&](hipStream_t st, const void* dq, const void* dk, const void* dv, float* dout) {
                                return run_device(variant, st, dq, dk, dv, bh, sq, sk, d, causal, nullptr, dout);
                            });
}

// ---------------------------------------------------------------------------
// Naive attention (src/naive.rs:14-75) on device pointers: scores, row
// softmax and PV kernels over a materialised [heads, seq_q, seq_k] buffer,
// heads taken in chunks whose buffer stays within kNaiveChunkBytes.
// ---------------------------------------------------------------------------
constexpr size_t kNaiveChunkBytes = size_t(8) << 30;

int launch_naive(int dev, const char* name, unsigned gx, unsigned gy, unsigned gz, NaiveParams* p,
                 hipStream_t stream) {
    hipFunction_t fn;
    int rc = get_function(dev, name, &fn);
    if (rc != FA_OK) return rc;
    void* args[] = {p};
    if (hipModuleLaunchKernel(fn, gx, gy, gz, 256, 1, 1, 0, stream, args, nullptr) != hipSuccess) {
        (void)hipGetLastError();
        return FA_ERR_LAUNCH;
    }
    return FA_OK;
}

int run_naive_device(hipStream_t stream, const float* q, const float* k, const float* v, size_t bh, size_t sq,
                     size_t sk, size_t d, int causal, int precision, float* out, float scale) {
    // The crate writes out = 0 when seq_len_k == 0 (every row's fill(0.0),
    // src/naive.rs:64); nothing is written when seq_len_q or d_head is 0.
    if (bh == 0 || sq == 0 || d == 0) return FA_OK;
    if (!q || !out || (sk > 0 && (!k || !v))) return FA_ERR_INVALID_ARG;
    if (precision != FA_NAIVE_F32 && precision != FA_NAIVE_F64) return FA_ERR_INVALID_ARG;
    const size_t imax = 0x7fffffff;
    if (sq > imax || sk > imax || d > imax || (sq + 63) / 64 > 65535 || (d + 63) / 64 > 65535)
        return FA_ERR_UNSUPPORTED;
    int dev;
    int rc = current_device(&dev);
    if (rc != FA_OK) return rc;
    rc = ensure_loaded(dev);
    if (rc != FA_OK) return rc;

    const bool f64 = precision == FA_NAIVE_F64;
    const size_t head_bytes = sq * sk * (f64 ? 8 : 4);
    // Score buffer: as many whole heads as fit in kNaiveChunkBytes and half
    // the free device memory (at least one); a head larger than half the
    // free memory is refused before anything is queued.
    const size_t half_free = head_bytes ? free_device_bytes() / 2 : 0;
    if (head_bytes && head_bytes > half_free) return FA_ERR_ALLOC;
    size_t chunk = head_bytes ? std::max<size_t>(1, std::min(kNaiveChunkBytes, half_free) / head_bytes) : bh;
    chunk = std::min({chunk, bh, (size_t)65535, imax / sq});
    void* s = nullptr;
    if (head_bytes) {
        if (hipMallocAsync(&s, chunk * head_bytes, stream) != hipSuccess) {
            (void)hipGetLastError();
            return FA_ERR_ALLOC;
        }
    }
    const char* sfx = f64 ? "f64" : "f32";
    std::string n_scores = std::string("fa_naive_scores_") + sfx, n_softmax = std::string("fa_naive_softmax_") + sfx,
                n_pv = std::string("fa_naive_pv_") + sfx;
    for (size_t h0 = 0; h0 < bh && rc == FA_OK; h0 += chunk) {
        const size_t nh = std::min(chunk, bh - h0);
        NaiveParams p;
        std::memset(&p, 0, sizeof(p));
        p.q = q + h0 * sq * d;
        p.k = sk ? k + h0 * sk * d : nullptr;
        p.v = sk ? v + h0 * sk * d : nullptr;
        p.out = out + h0 * sq * d;
        p.s = s;
        p.seq_q = static_cast<int>(sq);
        p.seq_k = static_cast<int>(sk);
        p.d = static_cast<int>(d);
        p.causal = causal ? 1 : 0;
        p.scale_f = 1.0f / std::sqrt(static_cast<float>(d));   // src/naive.rs:29
        p.scale_d = 1.0 / std::sqrt(static_cast<double>(d));
        if (scale > 0.0f && std::isfinite(scale)) {
            p.scale_f = scale;
            p.scale_d = static_cast<double>(scale);
        }
        const unsigned gq = static_cast<unsigned>((sq + 63) / 64);
        if (sk > 0) {
            rc = launch_naive(dev, n_scores.c_str(), static_cast<unsigned>((sk + 63) / 64), gq,
                              static_cast<unsigned>(nh), &p, stream);
            if (rc == FA_OK)
                rc = launch_naive(dev, n_softmax.c_str(), static_cast<unsigned>(nh * sq), 1, 1, &p, stream);
        }
        if (rc == FA_OK)
            rc = launch_naive(dev, n_pv.c_str(), static_cast<unsigned>((d + 63) / 64), gq, static_cast<unsigned>(nh),
                              &p, stream);
    }
    if (s && hipFreeAsync(s, stream) != hipSuccess) {
        (void)hipGetLastError();
        if (rc == FA_OK) rc = FA_ERR_ALLOC;
    }
    return rc;
}

int single(int variant, const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
           size_t v_len, size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out, size_t out_len) {
    const int rc = check_single(q_len, k_len, v_len, out_len, sq, sk, d);
    if (rc != FA_OK) return rc;
    return run_host(variant, q, k, v, 1, sq, sk, d, cfg, out);
}

int multi(int variant, const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
          size_t v_len, size_t batch, size_t heads, size_t sq, size_t sk, size_t d, const fa_config* cfg,
          float* out, size_t out_len) {
    // multihead_dispatch's totals (src/common.rs:85-90)
    const size_t bh = batch * heads;
    if (q_len != bh * sq * d) return FA_ERR_Q_SHAPE;
    if (k_len != bh * sk * d) return FA_ERR_K_SHAPE;
    if (v_len != bh * sk * d) return FA_ERR_V_SHAPE;
    if (out_len != bh * sq * d) return FA_ERR_OUT_SHAPE;
    return run_host(variant, q, k, v, bh, sq, sk, d, cfg, out);
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

const char* fa_status_string(int status) {
    switch (status) {
        case FA_OK: return "ok";
        case FA_ERR_Q_SHAPE: return "q shape mismatch";
        case FA_ERR_K_SHAPE: return "k shape mismatch";
        case FA_ERR_V_SHAPE: return "v shape mismatch";
        case FA_ERR_OUT_SHAPE: return "out shape mismatch";
        case FA_ERR_INVALID_ARG: return "invalid argument";
        case FA_ERR_UNSUPPORTED: return "unsupported shape (d_head > 256 with 16-bit inputs or split-KV, d_head > 2048 with a stream split or split count, or size beyond 32-bit indexing)";
        case FA_ERR_NO_DEVICE: return "no HIP device available";
        case FA_ERR_MODULE: return "cannot load the gfx950 code object (fa_kernels.hsaco / FA_HIP_MODULE)";
        case FA_ERR_ALLOC: return "device allocation failed";
        case FA_ERR_LAUNCH: return "kernel launch failed";
        case FA_ERR_COPY: return "host/device copy failed";
        case FA_ERR_SCRATCH: return "split workspace larger than the 64 MiB no-alloc scratch, or scratch unavailable";
        default: return "unknown status";
    }
}

fa_config fa_config_default(void) {
    fa_config c;
    c.block_size_q = 64;
    c.block_size_kv = 128;
    c.causal = 0;
    return c;
}

int fa_init(void) {
    int dev;
    const int rc = current_device(&dev);
    if (rc != FA_OK) return rc;
    return ensure_loaded(dev);
}

int fa_v1(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len, size_t sq,
          size_t sk, size_t d, const fa_config* cfg, float* out, size_t out_len) {
    return single(1, q, q_len, k, k_len, v, v_len, sq, sk, d, cfg, out, out_len);
}
int fa_v2(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len, size_t sq,
          size_t sk, size_t d, const fa_config* cfg, float* out, size_t out_len) {
    return single(2, q, q_len, k, k_len, v, v_len, sq, sk, d, cfg, out, out_len);
}
int fa_v3(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len, size_t sq,
          size_t sk, size_t d, const fa_config* cfg, float* out, size_t out_len) {
    return single(3, q, q_len, k, k_len, v, v_len, sq, sk, d, cfg, out, out_len);
}
int fa_attention(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
                 size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out, size_t out_len) {
    return single(2, q, q_len, k, k_len, v, v_len, sq, sk, d, cfg, out, out_len);
}

int fa_multihead_v1(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
                    size_t batch, size_t heads, size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out,
                    size_t out_len) {
    return multi(1, q, q_len, k, k_len, v, v_len, batch, heads, sq, sk, d, cfg, out, out_len);
}
int fa_multihead_v2(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
                    size_t batch, size_t heads, size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out,
                    size_t out_len) {
    return multi(2, q, q_len, k, k_len, v, v_len, batch, heads, sq, sk, d, cfg, out, out_len);
}
int fa_multihead_v3(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
                    size_t batch, size_t heads, size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out,
                    size_t out_len) {
    return multi(3, q, q_len, k, k_len, v, v_len, batch, heads, sq, sk, d, cfg, out, out_len);
}
int fa_attention_multihead(const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                           size_t v_len, size_t batch, size_t heads, size_t sq, size_t sk, size_t d,
                           const fa_config* cfg, float* out, size_t out_len) {
    return multi(2, q, q_len, k, k_len, v, v_len, batch, heads, sq, sk, d, cfg, out, out_len);
}

int fa_device_v1(void* stream, const float* q, const float* k, const float* v, size_t batch, size_t heads,
                 size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out) {
    return run_device(1, static_cast<hipStream_t>(stream), q, k, v, batch * heads, sq, sk, d,
                      cfg ? cfg->causal : 0, nullptr, out);
}
int fa_device_v2(void* stream, const float* q, const float* k, const float* v, size_t batch, size_t heads,
                 size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out) {
    return run_device(2, static_cast<hipStream_t>(stream), q, k, v, batch * heads, sq, sk, d,
                      cfg ? cfg->causal : 0, nullptr, out);
}
int fa_device_v3(void* stream, const float* q, const float* k, const float* v, size_t batch, size_t heads,
                 size_t sq, size_t sk, size_t d, const fa_config* cfg, float* out) {
    return run_device(3, static_cast<hipStream_t>(stream), q, k, v, batch * heads, sq, sk, d,
                      cfg ? cfg->causal : 0, nullptr, out);
}

int fa_naive_attention(const float* q, size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
                       size_t sq, size_t sk, size_t d, int causal, float* out, size_t out_len) {
    // assert_eq! order of src/naive.rs:24-27
    int rc = check_single(q_len, k_len, v_len, out_len, sq, sk, d);
    if (rc != FA_OK) return rc;
    if (sq == 0 || d == 0) return FA_OK;
    if (!q || !out || (sk > 0 && (!k || !v))) return FA_ERR_INVALID_ARG;
    return with_host_slices(q, k, v, sizeof(float), 1, sq, sk, d, out,
                            [&](hipStream_t st, const void* dq, const void* dk, const void* dv, float* dout) {
                                return run_naive_device(st, static_cast<const float*>(dq), static_cast<const float*>(dk),
                                                        static_cast<const float*>(dv), 1, sq, sk, d, causal,
                                                        FA_NAIVE_F32, dout, 0.0f);
                            });
}

int fa_naive_device(void* stream, const float* q, const float* k, const float* v, size_t batch, size_t heads,
                    size_t sq, size_t sk, size_t d, int causal, int precision, float* out) {
    return run_naive_device(static_cast<hipStream_t>(stream), q, k, v, batch * heads, sq, sk, d, causal, precision,
                            out, 0.0f);
}

int fa_device_ex(int variant, void* stream, const float* q, const float* k, const float* v, size_t batch,
                 size_t heads, size_t sq, size_t sk, size_t d, const fa_config* cfg, const fa_launch_opts* opts,
                 float* out) {
    if (variant < 1 || variant > 3) return FA_ERR_INVALID_ARG;
    if (opts && opts->dtype != FA_DTYPE_F32) return FA_ERR_INVALID_ARG;   // 16-bit inputs: fa_device_lp
    return run_device(variant, static_cast<hipStream_t>(stream), q, k, v, batch * heads, sq, sk, d,
                      cfg ? cfg->causal : 0, opts, out);
}

int fa_release_stream_workspace(void* stream) {
    int dev;
    int rc = current_device(&dev);
    if (rc != FA_OK) return rc;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    DeviceState& s = g_dev[dev];
    // Take the stream's buffers out of the table under the lock, then drain
    // the stream and free them without it, so split calls on other streams
    // of this device do not wait for this stream.
    std::vector<void*> bufs;
    {
        std::lock_guard<std::mutex> lock(s.ws_mu);
        auto it = s.ws.find(workspace_key(st));
        if (it == s.ws.end()) return FA_OK;
        bufs = std::move(it->second.retired);
        bufs.push_back(it->second.ptr);
        s.ws.erase(it);
    }
    // Work queued on the stream may still use the buffers.
    if (hipStreamSynchronize(st) != hipSuccess) {
        (void)hipGetLastError();
        return FA_ERR_COPY;   // the buffers stay allocated (never reused) rather than freed under work
    }
    rc = FA_OK;
    for (void* p : bufs)
        if (p && hipFree(p) != hipSuccess) {
            (void)hipGetLastError();
            rc = FA_ERR_ALLOC;
        }
    return rc;
}

int fa_device_ex_noalloc(int variant, void* stream, const float* q, const float* k, const float* v, size_t batch,
                         size_t heads, size_t sq, size_t sk, size_t d, const fa_config* cfg,
                         const fa_launch_opts* opts, float* out) {
    if (variant < 1 || variant > 3) return FA_ERR_INVALID_ARG;
    if (opts && opts->dtype != FA_DTYPE_F32) return FA_ERR_INVALID_ARG;
    return run_device(variant, static_cast<hipStream_t>(stream), q, k, v, batch * heads, sq, sk, d,
                      cfg ? cfg->causal : 0, opts, out, /*noalloc=*/true);
}

int fa_device_lp(int dtype, void* stream, const void* q, const void* k, const void* v, size_t batch, size_t heads,
                 size_t sq, size_t sk, size_t d, const fa_config* cfg, const fa_launch_opts* opts, float* out) {
    if (dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F16) return FA_ERR_INVALID_ARG;
    fa_launch_opts o = opts ? *opts : fa_launch_opts{0.0f, FA_PATH_AUTO, 0, dtype};
    o.dtype = dtype;
    return run_device(3, static_cast<hipStream_t>(stream), q, k, v, batch * heads, sq, sk, d, cfg ? cfg->causal : 0,
                      &o, out);
}

int fa_multihead_lp(int dtype, const void* q, size_t q_len, const void* k, size_t k_len, const void* v,
                    size_t v_len, size_t batch, size_t heads, size_t sq, size_t sk, size_t d, const fa_config* cfg,
                    float* out, size_t out_len) {
    if (dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F16) return FA_ERR_INVALID_ARG;
    const size_t bh = batch * heads;
    if (q_len != bh * sq * d) return FA_ERR_Q_SHAPE;
    if (k_len != bh * sk * d) return FA_ERR_K_SHAPE;
    if (v_len != bh * sk * d) return FA_ERR_V_SHAPE;
    if (out_len != bh * sq * d) return FA_ERR_OUT_SHAPE;
    if (bh == 0 || sq == 0 || sk == 0 || d == 0) return FA_OK;   // out untouched
    if (!q || !k || !v || !out) return FA_ERR_INVALID_ARG;
    if (d > (size_t)kMaxDNarrow) return FA_ERR_UNSUPPORTED;   // before any copy: the 16-bit kernels stop at 256
    const int causal = cfg ? cfg->causal : 0;
    const fa_launch_opts o{0.0f, FA_PATH_AUTO, 0, dtype};
    return with_host_slices(q, k, v, 2, bh, sq, sk, d, out,
                            [&](hipStream_t st, const void* dq, const void* dk, const void* dv, float* dout) {
                                return run_device(3, st, dq, dk, dv, bh, sq, sk, d, causal, &o, dout);
                            });
}

int fa_describe_launch(int variant, size_t batch, size_t heads, size_t sq, size_t sk, size_t d, int causal,
                       const fa_launch_opts* opts, char* buf, size_t buf_len) {
    int num_cus = 256;
    int n = 0, dev = 0;
    if (hipGetDeviceCount(&n) == hipSuccess && n > 0 && hipGetDevice(&dev) == hipSuccess) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
            num_cus = prop.multiProcessorCount;
    } else {
        (void)hipGetLastError();
    }
    const size_t bh = batch * heads;
    std::string text;
    int rc = FA_OK;
    if (bh == 0 || sq == 0 || sk == 0 || d == 0) {
        text = "none";
    } else {
        Plan plan;
        // Alignment is assumed (device allocations are 256-byte aligned).
        static const float dummy[4] __attribute__((aligned(16))) = {0, 0, 0, 0};
        rc = make_plan(variant, dummy, dummy, dummy, dummy, bh, sq, sk, d, causal, opts, num_cus, &plan);
        if (rc == FA_OK) {
            char tmp[256];
            std::snprintf(tmp, sizeof(tmp), "%s grid=%ux%ux%u block=%u", plan.first.name.c_str(), plan.first.gx,
                          plan.first.gy, plan.first.gz, plan.first.bx);
            text = tmp;
            if (plan.p.two_blocks) text += " two_blocks";
            if (plan.split) {
                std::snprintf(tmp, sizeof(tmp), "; %s grid=%ux%ux%u block=%u; splits=%d", plan.second.name.c_str(),
                              plan.second.gx, plan.second.gy, plan.second.gz, plan.second.bx, plan.p.num_splits);
                text += tmp;
                if (plan.p.stream_per > 0) {
                    std::snprintf(tmp, sizeof(tmp), " stream_per=%lld", plan.p.stream_per);
                    text += tmp;
                } else if (plan.p.split_len > 0) {
                    std::snprintf(tmp, sizeof(tmp), " split_len=%d", plan.p.split_len);
                    text += tmp;
                }
                std::snprintf(tmp, sizeof(tmp), " workspace=%zu", plan.ws_floats * sizeof(float));
                text += tmp;
            }
        }
    }
    if (buf && buf_len > 0) {
        std::strncpy(buf, text.c_str(), buf_len - 1);
        buf[buf_len - 1] = '\0';
    }
    return rc;
}

constexpr unsigned kProbeMaxIters = 1u << 20;

int fa_probe_launch(int kind, void* stream, void* buf, size_t bytes, unsigned iters, double* work) {
    if (kind < FA_PROBE_MFMA_F32_32X32X2 || kind > FA_PROBE_READ || !buf || !work) return FA_ERR_INVALID_ARG;
    if ((reinterpret_cast<uintptr_t>(buf) & 15u) != 0) return FA_ERR_INVALID_ARG;
    const bool stream_probe = kind == FA_PROBE_COPY || kind == FA_PROBE_READ;
    // argument checks that need no device come first
    // (an MFMA probe takes about a millisecond per 1,000 iterations: the cap keeps a launch near a second)
    if (stream_probe ? bytes / 32 == 0 : (iters == 0 || iters > kProbeMaxIters)) return FA_ERR_INVALID_ARG;
    int dev;
    int rc = current_device(&dev);
    if (rc != FA_OK) return rc;
    rc = ensure_loaded(dev);
    if (rc != FA_OK) return rc;
    static const char* const names[] = {"fa_probe_mfma_f32_32x32x2", "fa_probe_mfma_f32_16x16x4",
                                        "fa_probe_mfma_bf16_16x16x32", "fa_probe_copy",
                                        "fa_probe_mfma_bf16_32x32x16", "fa_probe_read"};
    const unsigned cus = static_cast<unsigned>(g_dev[dev].num_cus);
    ProbeParams pp{static_cast<float*>(buf), 0, iters};
    unsigned gx;
    if (stream_probe) {
        // the first half of the buffer in whole 16-byte elements: the copy's
        // source (its destination is the second half), or the read's data
        pp.n16 = bytes / 32;
        gx = 4 * cus;
        *work = (kind == FA_PROBE_COPY ? 32.0 : 16.0) * (double)pp.n16;   // bytes read (+ written)
    } else {
        // eight 4-wave workgroups per CU, two resident at a time; one
        // checksum float per wave
        gx = 8 * cus;
        if (bytes < (size_t)gx * 4 * sizeof(float)) return FA_ERR_INVALID_ARG;
        // FLOP per MFMA x independent chains per wave (index 3 is the copy)
        static const double per_iter[] = {2.0 * 32 * 32 * 2 * 4, 2.0 * 16 * 16 * 4 * 8, 2.0 * 16 * 16 * 32 * 16, 0.0,
                                          2.0 * 32 * 32 * 16 * 4};
        *work = (double)gx * 4.0 * (double)iters * per_iter[kind];
    }
    hipFunction_t fn;
    rc = get_function(dev, names[kind], &fn);
    if (rc != FA_OK) return rc;
    void* args[] = {&pp};
    if (hipModuleLaunchKernel(fn, gx, 1, 1, 256, 1, 1, 0, static_cast<hipStream_t>(stream), args, nullptr) !=
        hipSuccess) {
        (void)hipGetLastError();
        return FA_ERR_LAUNCH;
    }
    return FA_OK;
}

}  // extern "C"
