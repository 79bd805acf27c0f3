"""bench.py's contract pieces that run without a GPU: the one-GPU guard and
the work/byte counts its roofline uses."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_work_and_byte_counts_follow_the_stated_formulas():
    # FLOPs = 4 B H S^2 D, halved when causal (the FA2 convention)
    assert bench.flops(32, 8, 2048, 128, False) == 4 * 32 * 8 * 2048 ** 2 * 128 == 549755813888
    assert bench.flops(128, 8, 2048, 128, True) == 2 * 128 * 8 * 2048 ** 2 * 128
    # bytes = Q, K, V read once, O written once (2 bytes each), + the fp32 LSE when non-causal
    assert bench.algo_bytes(32, 8, 2048, 128, False) == 8 * 32 * 8 * 2048 * 128 + 4 * 32 * 8 * 2048 == 538968064
    assert bench.algo_bytes(128, 8, 2048, 128, True) == 8 * 128 * 8 * 2048 * 128
    # a float8 V is read as one byte per element
    assert bench.algo_bytes(32, 8, 2048, 128, False, v_bytes=1) == 7 * 32 * 8 * 2048 * 128 + 4 * 32 * 8 * 2048
