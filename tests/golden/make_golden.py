"""Write the golden fixtures tests/golden/attention_golden.npz.

The reference ships no tensors (its golden, torch_npu.npu_fusion_attention,
needs an Ascend NPU), so the fixtures are computed here, independently of the
oracle under test: plain float64 loops over every query row (no torch, no
vectorised softmax), from seeded fp16 inputs.  Cases cover causal and
non-causal, several head dims and scales, N=1, and the one-hot / zero-scale
special cases.

    python tests/golden/make_golden.py
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "attention_golden.npz")

# (name, N, D, causal, sm_scale, seed)
CASES = [
    ("nc_n16_d16", 16, 16, False, 0.25, 11),
    ("c_n16_d16", 16, 16, True, 0.25, 12),
    ("nc_n24_d32", 24, 32, False, 0.5, 13),
    ("c_n24_d32", 24, 32, True, 0.5, 14),
    ("nc_n40_d64", 40, 64, False, 0.125, 15),
    ("c_n40_d64", 40, 64, True, 0.125, 16),
    ("c_n33_d16_scale2", 33, 16, True, 2.0, 17),
    ("nc_n1_d32", 1, 32, False, 0.5, 18),
    ("c_n1_d32", 1, 32, True, 0.5, 19),
    ("nc_n16_d16_scale0", 16, 16, False, 0.0, 20),
    ("c_n16_d16_scale0", 16, 16, True, 0.0, 21),
    ("nc_n12_d16_negscale", 12, 16, False, -0.7, 22),
]


def brute(q, k, v, causal, scale):
    n, d = q.shape
    out = np.zeros((n, d))
    lse = np.zeros(n)
    for i in range(n):
        keys = list(range(i + 1)) if causal else list(range(n))
        s = [scale * sum(float(q[i, t]) * float(k[j, t]) for t in range(d)) for j in keys]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        tot = math.fsum(w)
        lse[i] = mx + math.log(tot)
        for t in range(d):
            out[i, t] = math.fsum(wj * float(v[j, t]) for wj, j in zip(w, keys)) / tot
    return out, lse


def main():
    arrays = {}
    for name, n, d, causal, scale, seed in CASES:
        rng = np.random.default_rng(seed)
        q = rng.standard_normal((n, d)).astype(np.float16)
        k = rng.standard_normal((n, d)).astype(np.float16)
        v = rng.standard_normal((n, d)).astype(np.float16)
        o, lse = brute(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), causal, scale)
        arrays[name + "/q"] = q
        arrays[name + "/k"] = k
        arrays[name + "/v"] = v
        arrays[name + "/o"] = o
        arrays[name + "/lse"] = lse
        arrays[name + "/meta"] = np.array([n, d, int(causal), scale, seed], dtype=np.float64)
    # one-hot retrieval: key j aligned with query i only, large scale
    n, d = 16, 16
    q = np.zeros((n, d), np.float16)
    k = np.zeros((n, d), np.float16)
    perm = np.random.default_rng(7).permutation(n)
    for i in range(n):
        q[i, i] = 1.0
        k[perm[i], i] = 1.0
    v = np.random.default_rng(8).standard_normal((n, d)).astype(np.float16)
    o, lse = brute(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), False, 64.0)
    for key, arr in (("q", q), ("k", k), ("v", v), ("o", o), ("lse", lse)):
        arrays["onehot_n16/" + key] = arr
    arrays["onehot_n16/meta"] = np.array([n, d, 0, 64.0, 7], dtype=np.float64)
    arrays["onehot_n16/perm"] = perm
    np.savez_compressed(OUT, **arrays)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
