"""Write tests/golden/input_fingerprints.json: SHA-256 of the seeded fp16 Q, K, V
of the five BASELINE configurations (oracle.attention.make_inputs, seeds 1234 +
config index) and of the north-star non-causal shape (seed 1240), so a machine that regenerates them can tell whether its torch
draws the same inputs.  A mismatch is reported by the tests, it does not void
parity (the oracle is recomputed from the same inputs in the same run).

    python tests/golden/make_fingerprints.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as A  # noqa: E402

# name, Z, H, N, D, seed (the order of BASELINE.json's configs)
CONFIGS = [
    ("C1", 2, 8, 1024, 128, 1235),
    ("C2", 32, 8, 2048, 128, 1236),
    ("C3", 128, 8, 2048, 128, 1237),
    ("C4", 64, 8, 1024, 256, 1238),
    ("C5", 4, 16, 8192, 64, 1239),
    # the north-star non-causal shape (B=128 H=8 S=2048 D=128), timed by bench.py
    ("target-noncausal", 128, 8, 2048, 128, 1240),
]


def main():
    import torch

    out = {"torch": torch.__version__, "generator": "torch.Generator('cpu'), randn fp32 then fp16, q, k, v order",
           "configs": {}}
    for name, Z, H, N, D, seed in CONFIGS:
        q, k, v = A.make_inputs(Z, H, N, D, seed)
        out["configs"][name] = {"shape": [Z, H, N, D], "seed": seed, "sha256": A.fingerprint(q, k, v)}
        del q, k, v
        print(name, out["configs"][name]["sha256"], flush=True)
    with open(os.path.join(HERE, "input_fingerprints.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
