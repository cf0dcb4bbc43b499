// fa_cpp_caller.cpp -- a C++ program using the header-only mirror of the
// crate's API (flash-attention-cpu_amd/csrc/flash_attention.hpp) over
// libfa_hip.so: std::vector slices, FlashAttentionConfig, exceptions.
//
// Usage and file formats: as fa_c_caller.c, with the crate's names:
// entry 0 flash_attention, 1-3 flash_attention_v1..v3,
// 4 flash_attention_multihead, 5-7 flash_attention_multihead_v1..v3,
// 8 naive_attention.  A thrown Error writes its status.  After the cases a
// wrong q length must throw ShapeMismatch("q shape mismatch") and leave out
// untouched; prints "cpp-caller ok".
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <vector>

#include "flash_attention.hpp"

namespace fa = flash_attention;

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s cases.bin outputs.bin\n", argv[0]);
        return 2;
    }
    std::ifstream in(argv[1], std::ios::binary);
    std::ofstream out(argv[2], std::ios::binary);
    uint32_t magic = 0, count = 0;
    in.read(reinterpret_cast<char*>(&magic), 4);
    in.read(reinterpret_cast<char*>(&count), 4);
    if (!in || magic != 0x31434146u) return 2;
    for (uint32_t c = 0; c < count; ++c) {
        int64_t h[9];
        in.read(reinterpret_cast<char*>(h), sizeof(h));
        const std::size_t b = h[1], hd = h[2], sq = h[3], sk = h[4], d = h[5];
        std::vector<float> q(b * hd * sq * d), k(b * hd * sk * d), v(b * hd * sk * d), o(b * hd * sq * d, 12.5f);
        in.read(reinterpret_cast<char*>(q.data()), q.size() * sizeof(float));
        in.read(reinterpret_cast<char*>(k.data()), k.size() * sizeof(float));
        in.read(reinterpret_cast<char*>(v.data()), v.size() * sizeof(float));
        if (!in) return 2;
        fa::FlashAttentionConfig cfg;
        cfg.block_size_q = h[6];
        cfg.block_size_kv = h[7];
        cfg.causal = h[8] != 0;
        int32_t st = FA_OK;
        try {
            switch (h[0]) {
                case 0: fa::flash_attention(q, k, v, sq, sk, d, cfg, o); break;
                case 1: fa::flash_attention_v1(q, k, v, sq, sk, d, cfg, o); break;
                case 2: fa::flash_attention_v2(q, k, v, sq, sk, d, cfg, o); break;
                case 3: fa::flash_attention_v3(q, k, v, sq, sk, d, cfg, o); break;
                case 4: fa::flash_attention_multihead(q, k, v, b, hd, sq, sk, d, cfg, o); break;
                case 5: fa::flash_attention_multihead_v1(q, k, v, b, hd, sq, sk, d, cfg, o); break;
                case 6: fa::flash_attention_multihead_v2(q, k, v, b, hd, sq, sk, d, cfg, o); break;
                case 7: fa::flash_attention_multihead_v3(q, k, v, b, hd, sq, sk, d, cfg, o); break;
                case 8: fa::naive_attention(q, k, v, sq, sk, d, cfg.causal, o); break;
                default: return 2;
            }
        } catch (const fa::Error& e) {
            st = e.status();
        }
        out.write(reinterpret_cast<const char*>(&st), 4);
        out.write(reinterpret_cast<const char*>(o.data()), o.size() * sizeof(float));
    }
    out.close();

    std::vector<float> a(8, 0.0f), o2(8, 3.0f), shortq(7, 0.0f);
    bool threw = false;
    try {
        fa::flash_attention(shortq, a, a, 2, 2, 4, fa::FlashAttentionConfig(), o2);
    } catch (const fa::ShapeMismatch& e) {
        threw = std::strcmp(e.what(), "q shape mismatch") == 0 && e.status() == FA_ERR_Q_SHAPE;
    }
    if (!threw || o2[0] != 3.0f) {
        std::fprintf(stderr, "shape check failed\n");
        return 1;
    }
    std::printf("cpp-caller ok\n");
    return 0;
}
