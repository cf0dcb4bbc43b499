// flash_attention.hpp -- header-only C++ mirror of the reference crate's
// public API (amaye15/flash-attention-cpu, src/lib.rs:78-87) over the C ABI
// in include/fa_hip.h.
//
// Same names, argument order and meaning as the Rust functions:
//   flash_attention_v1/v2/v3(q, k, v, seq_len_q, seq_len_k, d_head, config, out)
//   flash_attention_multihead_v1/v2/v3(q, k, v, batch, heads, seq_len_q,
//                                      seq_len_k, d_head, config, out)
//   flash_attention / flash_attention_multihead  (aliases of v2)
// Rust slices become Slice / MutSlice views (constructible from std::vector
// or pointer + length).  Where the crate panics on a shape mismatch
// (src/common.rs:51-54) these throw ShapeMismatch with the same message;
// other failures (no device, code object missing, ...) throw Error.
// Link with -lfa_hip.
#ifndef FLASH_ATTENTION_HPP
#define FLASH_ATTENTION_HPP

#include <cstddef>
#include <stdexcept>
#include <string>
#include <vector>

#include "fa_hip.h"

namespace flash_attention {

// FlashAttentionConfig (src/common.rs:16-36).
struct FlashAttentionConfig {
    std::size_t block_size_q = 64;
    std::size_t block_size_kv = 128;
    bool causal = false;
};

struct Slice {
    const float* data;
    std::size_t size;
    Slice(const float* p, std::size_t n) : data(p), size(n) {}
    Slice(const std::vector<float>& v) : data(v.data()), size(v.size()) {}  // NOLINT(implicit)
};

struct MutSlice {
    float* data;
    std::size_t size;
    MutSlice(float* p, std::size_t n) : data(p), size(n) {}
    MutSlice(std::vector<float>& v) : data(v.data()), size(v.size()) {}  // NOLINT(implicit)
};

class Error : public std::runtime_error {
   public:
    Error(int status, const char* msg) : std::runtime_error(msg), status_(status) {}
    int status() const { return status_; }

   private:
    int status_;
};

// The crate's shape assert failed ("q shape mismatch", ...).
class ShapeMismatch : public Error {
   public:
    using Error::Error;
};

namespace detail {
inline fa_config to_c(const FlashAttentionConfig& c) {
    fa_config r;
    r.block_size_q = c.block_size_q;
    r.block_size_kv = c.block_size_kv;
    r.causal = c.causal ? 1 : 0;
    return r;
}
inline void check(int status) {
    if (status == FA_OK) return;
    if (status >= FA_ERR_Q_SHAPE && status <= FA_ERR_OUT_SHAPE) throw ShapeMismatch(status, fa_status_string(status));
    throw Error(status, fa_status_string(status));
}
using SingleFn = int (*)(const float*, size_t, const float*, size_t, const float*, size_t, size_t, size_t, size_t,
                         const fa_config*, float*, size_t);
using MultiFn = int (*)(const float*, size_t, const float*, size_t, const float*, size_t, size_t, size_t, size_t,
                        size_t, size_t, const fa_config*, float*, size_t);
inline void single(SingleFn f, Slice q, Slice k, Slice v, std::size_t sq, std::size_t sk, std::size_t d,
                   const FlashAttentionConfig& cfg, MutSlice out) {
    const fa_config c = to_c(cfg);
    check(f(q.data, q.size, k.data, k.size, v.data, v.size, sq, sk, d, &c, out.data, out.size));
}
inline void multi(MultiFn f, Slice q, Slice k, Slice v, std::size_t b, std::size_t h, std::size_t sq, std::size_t sk,
                  std::size_t d, const FlashAttentionConfig& cfg, MutSlice out) {
    const fa_config c = to_c(cfg);
    check(f(q.data, q.size, k.data, k.size, v.data, v.size, b, h, sq, sk, d, &c, out.data, out.size));
}
}  // namespace detail

// flash_attention_v1 -- src/v1.rs:51
inline void flash_attention_v1(Slice q, Slice k, Slice v, std::size_t seq_len_q, std::size_t seq_len_k,
                               std::size_t d_head, const FlashAttentionConfig& config, MutSlice out) {
    detail::single(fa_v1, q, k, v, seq_len_q, seq_len_k, d_head, config, out);
}
// flash_attention_v2 -- src/v2.rs:49
inline void flash_attention_v2(Slice q, Slice k, Slice v, std::size_t seq_len_q, std::size_t seq_len_k,
                               std::size_t d_head, const FlashAttentionConfig& config, MutSlice out) {
    detail::single(fa_v2, q, k, v, seq_len_q, seq_len_k, d_head, config, out);
}
// flash_attention_v3 -- src/v3.rs:61
inline void flash_attention_v3(Slice q, Slice k, Slice v, std::size_t seq_len_q, std::size_t seq_len_k,
                               std::size_t d_head, const FlashAttentionConfig& config, MutSlice out) {
    detail::single(fa_v3, q, k, v, seq_len_q, seq_len_k, d_head, config, out);
}
// flash_attention_multihead_v1 -- src/v1.rs:134
inline void flash_attention_multihead_v1(Slice q, Slice k, Slice v, std::size_t batch, std::size_t heads,
                                         std::size_t seq_len_q, std::size_t seq_len_k, std::size_t d_head,
                                         const FlashAttentionConfig& config, MutSlice out) {
    detail::multi(fa_multihead_v1, q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out);
}
// flash_attention_multihead_v2 -- src/v2.rs:132
inline void flash_attention_multihead_v2(Slice q, Slice k, Slice v, std::size_t batch, std::size_t heads,
                                         std::size_t seq_len_q, std::size_t seq_len_k, std::size_t d_head,
                                         const FlashAttentionConfig& config, MutSlice out) {
    detail::multi(fa_multihead_v2, q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out);
}
// flash_attention_multihead_v3 -- src/v3.rs:144
inline void flash_attention_multihead_v3(Slice q, Slice k, Slice v, std::size_t batch, std::size_t heads,
                                         std::size_t seq_len_q, std::size_t seq_len_k, std::size_t d_head,
                                         const FlashAttentionConfig& config, MutSlice out) {
    detail::multi(fa_multihead_v3, q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out);
}
// naive_attention -- src/naive.rs:14 (materialised scores, on the GPU)
inline void naive_attention(Slice q, Slice k, Slice v, std::size_t seq_len_q, std::size_t seq_len_k,
                            std::size_t d_head, bool causal, MutSlice out) {
    detail::check(fa_naive_attention(q.data, q.size, k.data, k.size, v.data, v.size, seq_len_q, seq_len_k, d_head,
                                     causal ? 1 : 0, out.data, out.size));
}
// Aliases of v2 -- src/lib.rs:86-87 (through the C ABI's own aliases)
inline void flash_attention(Slice q, Slice k, Slice v, std::size_t seq_len_q, std::size_t seq_len_k,
                            std::size_t d_head, const FlashAttentionConfig& config, MutSlice out) {
    detail::single(fa_attention, q, k, v, seq_len_q, seq_len_k, d_head, config, out);
}
inline void flash_attention_multihead(Slice q, Slice k, Slice v, std::size_t batch, std::size_t heads,
                                      std::size_t seq_len_q, std::size_t seq_len_k, std::size_t d_head,
                                      const FlashAttentionConfig& config, MutSlice out) {
    detail::multi(fa_attention_multihead, q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out);
}

}  // namespace flash_attention

#endif  // FLASH_ATTENTION_HPP
