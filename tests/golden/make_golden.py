"""Write the golden vectors in tests/golden/golden.npz.

The reference crate commits no golden vectors (its tests recompute the
expected output with naive_attention, src/naive.rs:14-75, or compare
variants), so these fixtures are produced here, independently of both the
CPU oracle and the HIP kernels: inputs from numpy's PCG64 generator, and the
expected output from textbook softmax attention evaluated in float64 numpy
(fa_testutil.attention_f64: scale 1/sqrt(d) computed in f32 as
src/v2.rs:171, causal mask j > i as src/naive.rs:37, rows with no visible
key -> 0 as src/naive.rs:54).

Shapes: BASELINE.json configs[0] (256 x 256, d 64, N(0,1), non-causal) and
the edge shapes of tests/correctness.rs (ragged, single row / key, odd d,
causal with block > seq, asymmetric causal, multihead), plus a small peaky
case (Q, K ~ N(0, 9)).

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from fa_testutil import attention_f64  # noqa: E402

CASES = [
    # name, bh, seq_q, seq_k, d, causal, dist
    ("config1_256x256_d64", 1, 256, 256, 64, False, "normal"),
    ("ragged_17x23_d32", 1, 17, 23, 32, False, "uniform"),
    ("single_1x1_d16", 1, 1, 1, 16, False, "uniform"),
    ("one_query_1x50_d33", 1, 1, 50, 33, False, "uniform"),
    ("one_key_50x1_d33", 1, 50, 1, 33, False, "uniform"),
    ("ragged_97x131_d17", 1, 97, 131, 17, False, "uniform"),
    ("causal_97x97_d33", 1, 97, 97, 33, True, "uniform"),
    ("causal_5x5_d8", 1, 5, 5, 8, True, "uniform"),
    ("causal_asym_10x40_d32", 1, 10, 40, 32, True, "uniform"),
    ("causal_200x200_d128", 1, 200, 200, 128, True, "uniform"),
    ("multihead_2x3_37x50_d16", 6, 37, 50, 16, True, "uniform"),
    ("peaky_64x48_d256", 2, 64, 48, 256, False, "peaky"),
]


def make():
    out = {}
    for idx, (name, bh, sq, sk, d, causal, dist) in enumerate(CASES):
        rng = np.random.default_rng(1000 + idx)
        if dist == "normal":
            q = rng.standard_normal(bh * sq * d).astype(np.float32)
            k = rng.standard_normal(bh * sk * d).astype(np.float32)
            v = rng.standard_normal(bh * sk * d).astype(np.float32)
        elif dist == "peaky":
            q = (3.0 * rng.standard_normal(bh * sq * d)).astype(np.float32)
            k = (3.0 * rng.standard_normal(bh * sk * d)).astype(np.float32)
            v = rng.uniform(-1, 1, bh * sk * d).astype(np.float32)
        else:
            q = rng.uniform(-1, 1, bh * sq * d).astype(np.float32)
            k = rng.uniform(-1, 1, bh * sk * d).astype(np.float32)
            v = rng.uniform(-1, 1, bh * sk * d).astype(np.float32)
        exp = np.concatenate([
            attention_f64(q[h * sq * d:(h + 1) * sq * d], k[h * sk * d:(h + 1) * sk * d],
                          v[h * sk * d:(h + 1) * sk * d], sq, sk, d, causal) for h in range(bh)])
        out[f"{name}__shape"] = np.array([bh, sq, sk, d, int(causal)], dtype=np.int64)
        out[f"{name}__q"] = q
        out[f"{name}__k"] = k
        out[f"{name}__v"] = v
        out[f"{name}__out"] = exp.astype(np.float32)   # float64 result rounded once
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)


def load():
    """{name: (bh, seq_q, seq_k, d, causal, q, k, v, expected)}."""
    z = np.load(os.path.join(HERE, "golden.npz"))
    cases = {}
    for key in z.files:
        if key.endswith("__shape"):
            name = key[:-7]
            bh, sq, sk, d, causal = (int(x) for x in z[key])
            cases[name] = (bh, sq, sk, d, bool(causal), z[name + "__q"], z[name + "__k"], z[name + "__v"],
                           z[name + "__out"])
    return cases


if __name__ == "__main__":
    make()
    print("wrote", os.path.join(HERE, "golden.npz"))
