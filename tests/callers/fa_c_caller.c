/*
 * fa_c_caller.c -- a plain C program calling libfa_hip.so through
 * include/fa_hip.h, as a foreign caller (the crate's users, via FFI) would.
 *
 * Usage: fa_c_caller <cases.bin> <outputs.bin>
 *
 * cases.bin:   uint32 magic 0x31434146 ("FAC1"), uint32 case count, then per
 *              case 9 int64 (entry, batch, heads, seq_q, seq_k, d_head,
 *              block_size_q, block_size_kv, causal) and the f32 Q, K, V
 *              ([batch*heads, seq, d_head] each).
 * outputs.bin: per case an int32 status and batch*heads*seq_q*d_head f32
 *              of out (pre-filled with 12.5, so untouched outputs show).
 * entry: 0 fa_attention, 1-3 fa_v1..fa_v3, 4 fa_attention_multihead,
 *        5-7 fa_multihead_v1..v3, 8 fa_naive_attention.
 * After the cases it checks that a wrong q length returns FA_ERR_Q_SHAPE
 * and leaves out untouched, and prints "c-caller ok".
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "fa_hip.h"

static int read_all(FILE* f, void* p, size_t bytes) { return fread(p, 1, bytes, f) == bytes; }

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s cases.bin outputs.bin\n", argv[0]);
        return 2;
    }
    FILE* in = fopen(argv[1], "rb");
    FILE* out = fopen(argv[2], "wb");
    if (!in || !out) return 2;
    uint32_t magic = 0, count = 0;
    if (!read_all(in, &magic, 4) || !read_all(in, &count, 4) || magic != 0x31434146u) return 2;
    for (uint32_t c = 0; c < count; ++c) {
        int64_t h[9];
        if (!read_all(in, h, sizeof(h))) return 2;
        const size_t bh = (size_t)(h[1] * h[2]), sq = (size_t)h[3], sk = (size_t)h[4], d = (size_t)h[5];
        const size_t nq = bh * sq * d, nk = bh * sk * d;
        float* q = malloc((nq ? nq : 1) * sizeof(float));
        float* k = malloc((nk ? nk : 1) * sizeof(float));
        float* v = malloc((nk ? nk : 1) * sizeof(float));
        float* o = malloc((nq ? nq : 1) * sizeof(float));
        if (!q || !k || !v || !o) return 3;
        if (!read_all(in, q, nq * sizeof(float)) || !read_all(in, k, nk * sizeof(float)) ||
            !read_all(in, v, nk * sizeof(float)))
            return 2;
        for (size_t i = 0; i < nq; ++i) o[i] = 12.5f;
        fa_config cfg = fa_config_default();
        cfg.block_size_q = (size_t)h[6];
        cfg.block_size_kv = (size_t)h[7];
        cfg.causal = (uint8_t)(h[8] != 0);
        int st;
        switch (h[0]) {
            case 0: st = fa_attention(q, nq, k, nk, v, nk, sq, sk, d, &cfg, o, nq); break;
            case 1: st = fa_v1(q, nq, k, nk, v, nk, sq, sk, d, &cfg, o, nq); break;
            case 2: st = fa_v2(q, nq, k, nk, v, nk, sq, sk, d, &cfg, o, nq); break;
            case 3: st = fa_v3(q, nq, k, nk, v, nk, sq, sk, d, &cfg, o, nq); break;
            case 4:
                st = fa_attention_multihead(q, nq, k, nk, v, nk, (size_t)h[1], (size_t)h[2], sq, sk, d, &cfg, o, nq);
                break;
            case 5: st = fa_multihead_v1(q, nq, k, nk, v, nk, (size_t)h[1], (size_t)h[2], sq, sk, d, &cfg, o, nq); break;
            case 6: st = fa_multihead_v2(q, nq, k, nk, v, nk, (size_t)h[1], (size_t)h[2], sq, sk, d, &cfg, o, nq); break;
            case 7: st = fa_multihead_v3(q, nq, k, nk, v, nk, (size_t)h[1], (size_t)h[2], sq, sk, d, &cfg, o, nq); break;
            case 8: st = fa_naive_attention(q, nq, k, nk, v, nk, sq, sk, d, cfg.causal, o, nq); break;
            default: return 2;
        }
        const int32_t st32 = st;
        fwrite(&st32, 4, 1, out);
        fwrite(o, sizeof(float), nq, out);
        free(q);
        free(k);
        free(v);
        free(o);
    }
    fclose(in);
    fclose(out);

    /* the crate's assert on q's length (src/common.rs:51) as a status */
    float a[8] = {0}, o2[8];
    for (int i = 0; i < 8; ++i) o2[i] = 3.0f;
    const int st = fa_attention(a, 7, a, 8, a, 8, 2, 2, 4, NULL, o2, 8);
    if (st != FA_ERR_Q_SHAPE || o2[0] != 3.0f) {
        fprintf(stderr, "shape check: status %d (%s)\n", st, fa_status_string(st));
        return 1;
    }
    printf("c-caller ok\n");
    return 0;
}
