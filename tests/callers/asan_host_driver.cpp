// asan_host_driver.cpp -- exercises the CPU-side paths of the host library
// (flash-attention-cpu_amd/csrc/fa_host.cpp, compiled into this program with
// AddressSanitizer and UndefinedBehaviorSanitizer): the launch planner over a
// sweep of shapes, paths, split counts and dtypes (fa_describe_launch), the
// shape checks of every host-slice entry point, zero-sized dimensions, status
// strings, argument errors, and -- when no GPU is visible -- the no-device
// path of every compute entry point.  Nothing here launches a kernel.
//
// The device-global scratch array lives in fa_scratch.hip (a HIP source);
// this host-only build replaces its two lookup functions with stubs that
// report it unavailable.
#include <cstdio>
#include <cstring>
#include <vector>

#include "fa_hip.h"
#include "fa_scratch.h"

int fa_scratch_init(int) { return FA_ERR_SCRATCH; }
void* fa_scratch_ptr(int) { return nullptr; }

static int failures = 0;
#define CHECK(cond, ...)                                 \
    do {                                                 \
        if (!(cond)) {                                   \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);           \
            std::fprintf(stderr, "\n");                  \
            ++failures;                                  \
        }                                                \
    } while (0)

static bool untouched(const std::vector<float>& o, float v) {
    for (float x : o)
        if (x != v) return false;
    return true;
}

int main() {
    const bool device = fa_init() == FA_OK;

    // status strings and the default config
    for (int s = -3; s < 40; ++s) CHECK(fa_status_string(s) && std::strlen(fa_status_string(s)) > 0, "status %d", s);
    const fa_config def = fa_config_default();
    CHECK(def.block_size_q == 64 && def.block_size_kv == 128 && def.causal == 0, "default config");

    // planner sweep
    const size_t bhs[] = {1, 3, 32, 4096};
    const size_t seqs[] = {1, 2, 3, 4, 5, 15, 16, 17, 63, 64, 65, 127, 128, 129, 256, 1000, 2048, 16384, 32768};
    const size_t ds[] = {1, 3, 4, 8, 17, 31, 32, 33, 64, 100, 127, 128, 129, 200, 255, 256, 257, 512, 513, 1000, 1024, 1025};
    const int splits[] = {0, 1, 2, 3, 16, 1024, 1025};
    char buf[512];
    long plans = 0;
    // every (variant, bh, seq_q, seq_k, d) with one (path, dtype, split
    // count, causal) chosen from the index, so all of them recur
    for (int variant = 0; variant <= 4; ++variant)
        for (size_t bh : bhs)
            for (size_t sq : seqs)
                for (size_t sk : seqs)
                    for (size_t d : ds) {
                        const long i = plans;
                        const int path = (int)(i % 6) - 1, dtype = (int)((i / 6) % 4);
                        const int ns = splits[(i / 24) % 7], causal = (int)((i / 168) % 2);
                        fa_launch_opts o{0.0f, path, ns, dtype};
                        std::memset(buf, 'x', sizeof(buf));
                        const int rc = fa_describe_launch(variant, 1, bh, sq, sk, d, causal, &o, buf, sizeof(buf));
                        CHECK(rc >= FA_OK && rc <= FA_ERR_SCRATCH, "rc %d", rc);
                        CHECK(std::memchr(buf, 0, sizeof(buf)) != nullptr, "unterminated description");
                        ++plans;
                    }
    // truncation of the description buffer
    for (size_t len : {(size_t)1, (size_t)2, (size_t)8, (size_t)33}) {
        std::vector<char> small(len, 'x');
        fa_describe_launch(2, 1, 32, 1, 32768, 128, 0, nullptr, small.data(), small.size());
        CHECK(small[len - 1] == '\0', "truncation at %zu", len);
    }
    fa_describe_launch(2, 1, 32, 1, 32768, 128, 0, nullptr, nullptr, 0);

    // shape checks: q, k, v, out in that order; out untouched
    const size_t sq = 5, sk = 7, d = 6;
    std::vector<float> q(sq * d, 1.0f), k(sk * d, 1.0f), v(sk * d, 1.0f), o(sq * d, 3.5f);
    typedef int (*Single)(const float*, size_t, const float*, size_t, const float*, size_t, size_t, size_t, size_t,
                          const fa_config*, float*, size_t);
    const Single singles[] = {fa_v1, fa_v2, fa_v3, fa_attention};
    for (Single f : singles) {
        CHECK(f(q.data(), q.size() - 1, k.data(), k.size() - 1, v.data(), 0, sq, sk, d, nullptr, o.data(), 1) ==
                  FA_ERR_Q_SHAPE, "q first");
        CHECK(f(q.data(), q.size(), k.data(), k.size() + 1, v.data(), 0, sq, sk, d, nullptr, o.data(), 1) ==
                  FA_ERR_K_SHAPE, "k second");
        CHECK(f(q.data(), q.size(), k.data(), k.size(), v.data(), 3, sq, sk, d, nullptr, o.data(), 1) ==
                  FA_ERR_V_SHAPE, "v third");
        CHECK(f(q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), sq, sk, d, &def, o.data(), 1) ==
                  FA_ERR_OUT_SHAPE, "out last");
        CHECK(untouched(o, 3.5f), "out touched by a shape error");
        // zero-sized dims: FA_OK, untouched
        CHECK(f(nullptr, 0, k.data(), k.size(), v.data(), v.size(), 0, sk, d, nullptr, nullptr, 0) == FA_OK, "sq 0");
        CHECK(f(q.data(), 0, nullptr, 0, nullptr, 0, sq, 0, 0, nullptr, o.data(), 0) == FA_OK, "d 0");
    }
    typedef int (*Multi)(const float*, size_t, const float*, size_t, const float*, size_t, size_t, size_t, size_t,
                         size_t, size_t, const fa_config*, float*, size_t);
    const Multi multis[] = {fa_multihead_v1, fa_multihead_v2, fa_multihead_v3, fa_attention_multihead};
    for (Multi f : multis) {
        CHECK(f(q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), 2, 3, sq, sk, d, nullptr, o.data(),
                o.size()) == FA_ERR_Q_SHAPE, "multihead q");
        CHECK(f(nullptr, 0, nullptr, 0, nullptr, 0, 0, 3, sq, sk, d, nullptr, nullptr, 0) == FA_OK, "batch 0");
    }
    CHECK(fa_multihead_lp(FA_DTYPE_BF16, q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), 1, 1, sq, sk, 300,
                          nullptr, o.data(), o.size()) == FA_ERR_Q_SHAPE, "lp q");
    CHECK(fa_multihead_lp(7, q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), 1, 1, sq, sk, d, nullptr,
                          o.data(), o.size()) == FA_ERR_INVALID_ARG, "lp dtype");
    CHECK(fa_naive_attention(q.data(), 2, k.data(), k.size(), v.data(), v.size(), sq, sk, d, 0, o.data(), o.size()) ==
              FA_ERR_Q_SHAPE, "naive q");
    CHECK(untouched(o, 3.5f), "out touched");

    // argument errors before any device work
    fa_launch_opts bad{0.0f, 9, 0, 0};
    CHECK(fa_device_ex(7, nullptr, q.data(), k.data(), v.data(), 1, 1, sq, sk, d, nullptr, nullptr, o.data()) ==
              FA_ERR_INVALID_ARG, "variant");
    CHECK(fa_device_ex_noalloc(0, nullptr, q.data(), k.data(), v.data(), 1, 1, sq, sk, d, nullptr, nullptr,
                               o.data()) == FA_ERR_INVALID_ARG, "noalloc variant");
    CHECK(fa_device_lp(0, nullptr, q.data(), k.data(), v.data(), 1, 1, sq, sk, d, nullptr, nullptr, o.data()) ==
              FA_ERR_INVALID_ARG, "lp dtype");
    CHECK(fa_describe_launch(2, 1, 1, sq, sk, d, 0, &bad, buf, sizeof(buf)) == FA_ERR_INVALID_ARG, "bad path");

    // no device: every compute entry point fails loudly, out untouched
    if (!device) {
        for (Single f : singles)
            CHECK(f(q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), sq, sk, d, nullptr, o.data(),
                    o.size()) == FA_ERR_NO_DEVICE, "single no device");
        for (Multi f : multis)
            CHECK(f(q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), 1, 1, sq, sk, d, nullptr, o.data(),
                    o.size()) == FA_ERR_NO_DEVICE, "multi no device");
        CHECK(fa_device_v2(nullptr, q.data(), k.data(), v.data(), 1, 1, sq, sk, d, nullptr, o.data()) ==
                  FA_ERR_NO_DEVICE, "device no device");
        CHECK(fa_device_ex_noalloc(2, nullptr, q.data(), k.data(), v.data(), 1, 1, sq, sk, d, nullptr, nullptr,
                                   o.data()) == FA_ERR_NO_DEVICE, "noalloc no device");
        CHECK(fa_naive_attention(q.data(), q.size(), k.data(), k.size(), v.data(), v.size(), sq, sk, d, 1, o.data(),
                                 o.size()) == FA_ERR_NO_DEVICE, "naive no device");
        CHECK(fa_release_stream_workspace(nullptr) == FA_ERR_NO_DEVICE, "release no device");
        CHECK(untouched(o, 3.5f), "out touched without a device");
    }
    std::printf("plans=%ld failures=%d\n", plans, failures);
    if (failures == 0) std::printf("asan-host ok\n");
    return failures ? 1 : 0;
}
