"""Benchmark of the FlashAttention-2 forward on one MI355X.

Prints ONE JSON line.  A step is one ``attention(q, k, v, causal, sm_scale,
BM, BN)`` call (the reference's public entry point) over the workload's
seeded synthetic Q/K/V, already resident in HBM.  ``value`` is the algorithmic
throughput 4*B*H*S^2*D (x0.5 causal) / time in TFLOP/s of the BASELINE workload
configs[1] (non-causal B=32 H=8 S=2048 D=128), timed as K back-to-back calls
between two HIP events on the stream the kernel is launched on.  The other
BASELINE configs and the north-star target shape are timed the same way and
reported under ``"configs"``.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]
                    [--calibrate-copy-mib M]

``--calibrate-copy-mib M`` adds one plain device-to-device copy of M MiB after
the timed work; under ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` it gives
the counter reading of a kernel with known traffic, which scales the readings
of the attention kernel to bytes.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ascend-rsfa_amd"))
sys.path.insert(0, ROOT)

METRIC = "FA2 fwd TFLOP/s + % fp16 MFMA peak (causal & non-causal), ms/call"
PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published
PEAK_HBM_GBS = 8000.0

# name, B, H, S, D, causal, sm_scale, seed[, V dtype]
CONFIGS = [
    ("C2", 32, 8, 2048, 128, False, 1 / math.sqrt(128), 1236),   # the `value`
    ("C3", 128, 8, 2048, 128, True, 0.5, 1237),
    ("target-noncausal", 128, 8, 2048, 128, False, 1 / math.sqrt(128), 1240),
    ("C4-noncausal", 64, 8, 1024, 256, False, 1 / 16, 1238),
    ("C4-causal", 64, 8, 1024, 256, True, 1 / 16, 1238),
    ("C5", 4, 16, 8192, 64, True, 1 / 8, 1239),
    ("C1", 2, 8, 1024, 128, True, 0.5, 1235),
    # the reference's fp8_v branch (flash_attention_forward.py:208-211): fp16 Q, K, O, float8 e5m2 V
    ("C2-v8e5m2", 32, 8, 2048, 128, False, 1 / math.sqrt(128), 1236, "e5m2"),
]
# HBM bytes per launch of the C2 kernel, from two rocprofv3 --pmc passes
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "fa_fwd_c2_traffic.txt")


def flops(B, H, S, D, causal):
    return 4.0 * B * H * S * S * D * (0.5 if causal else 1.0)


def algo_bytes(B, H, S, D, causal, v_bytes=2):
    # Q, K, V read once, O written once (fp16; V 1 byte when float8); non-causal
    # attention() also writes the fp32 row logsumexp M (reference 400-403)
    return (2.0 * 3 + v_bytes) * B * H * S * D + (0.0 if causal else 4.0 * B * H * S)


def time_config(F, torch, cfg, steps, warmup):
    name, B, H, S, D, causal, scale, seed = cfg[:8]
    v8 = len(cfg) > 8 and cfg[8] == "e5m2"
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    shape = (B, H, S, D)
    q = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).half()
    k = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32).half()
    v = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32)
    v = v.to(torch.float8_e5m2) if v8 else v.half()
    BM, BN = F.get_tiling(B, H, S, D, causal)
    for _ in range(warmup):
        F.attention(q, k, v, causal, scale, BM, BN)
    # attention() enqueues its kernel on the current stream: the events go there
    stream = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(steps):
        F.attention(q, k, v, causal, scale, BM, BN)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    fl = flops(B, H, S, D, causal)
    del q, k, v
    torch.cuda.empty_cache()
    return {
        "B": B, "H": H, "S": S, "D": D, "causal": causal, "sm_scale": scale, "tiling": [BM, BN],
        "ms_per_call": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
        "pct_peak": round(100.0 * fl / (ms * 1e-3) / 1e12 / PEAK_TFLOPS, 2),
        "hbm_gbs_algorithmic": round(algo_bytes(B, H, S, D, causal, 1 if v8 else 2) / (ms * 1e-3) / 1e9, 1),
        **({"v_dtype": "float8_e5m2"} if v8 else {}),
    }


def calibrate_copy(torch, mib):
    """One plain device copy of `mib` MiB (reads and writes mib MiB each)."""
    n = mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] calibration copy: {n} bytes read, {n} bytes written", file=sys.stderr, flush=True)


def cpu_baseline(torch, cfg, budget_s=10.0):
    """The reference's attention math (the oracle's fp32 closed form) on the host cores.

    Bounded sample: whole heads of the workload, repeated until about
    ``budget_s`` seconds of CPU time have run.
    """
    from oracle import attention as oracle

    name, B, H, S, D, causal, scale, seed = cfg
    threads = torch.get_num_threads()
    q, k, v = oracle.make_inputs(1, 1, S, D, seed)
    oracle.reference_attention(q, k, v, causal, scale)  # warmup
    t = time.perf_counter()
    oracle.reference_attention(q, k, v, causal, scale)
    one = max(time.perf_counter() - t, 1e-4)
    heads = max(1, min(B * H, int(budget_s / one)))
    q, k, v = oracle.make_inputs(1, heads, S, D, seed)
    reps = 0
    t = time.perf_counter()
    while True:
        oracle.reference_attention(q, k, v, causal, scale)
        reps += 1
        el = time.perf_counter() - t
        if el >= budget_s * 0.5 or reps >= 20:
            break
    fl = flops(1, heads, S, D, causal) * reps
    return {
        "value": round(fl / el / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"{reps} x {heads} of {B * H} heads of {name} (S={S}, D={D}, causal={causal}): the fp32 closed "
                  f"form softmax(QK^T*scale)V in PyTorch on {threads} host threads, {el:.1f} s; "
                  f"full S^2 computed even when causal; FLOPs counted as on the GPU",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # The GPU's clocks settle only after ~100 ms of sustained MFMA load (the
    # first launches run at boost clocks, then dip below the steady state):
    # the default warmup lets the timed steps see the steady state.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default=None, help="time only this config name")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the path shards by (batch, head) with no "
                                   "communication, so runs with --gpus N > 1 are not part of it"}))
        sys.exit(2)

    import torch

    from ascend_rsfa import _native
    from ascend_rsfa import flash_attention_forward as F

    if not os.path.exists(_native.library_path()):
        raise SystemExit(f"{_native.library_path()} is not built: run `python __graft_entry__.py build` first")
    torch.cuda.set_device(0)
    configs = [c for c in CONFIGS if args.only in (None, c[0])]
    results = {}
    for cfg in configs:
        results[cfg[0]] = time_config(F, torch, cfg, args.steps, args.warmup)
        print(f"[bench] {cfg[0]}: {results[cfg[0]]}", file=sys.stderr, flush=True)
    if args.calibrate_copy_mib:
        calibrate_copy(torch, args.calibrate_copy_mib)
    main_name = configs[0][0]
    r = results[main_name]
    cfg = configs[0]
    # average duration of one launch over the timed region (back-to-back launches)
    achieved = flops(*cfg[1:6]) / (r["ms_per_call"] * 1e-3) / 1e12
    traffic = None
    if main_name == "C2" and os.path.exists(PROFILE_TRAFFIC):
        with open(PROFILE_TRAFFIC) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    traffic = int(float(line.split(":", 1)[1]))
    line = {
        "metric": METRIC,
        "value": r["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_call"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded Q,K,V ~ N(0,1) fp16, resident in HBM",
        "config": {"workload": f"{main_name}: B={cfg[1]} H={cfg[2]} S={cfg[3]} D={cfg[4]} "
                               f"{'causal' if cfg[5] else 'non-causal'} sm_scale={cfg[6]:.6g}",
                   "layout": "[B,H,S,D]", "tiling": r["tiling"], "parallelism": "single GPU"},
        "pct_peak": r["pct_peak"],
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TFLOPS, 4), "traffic": traffic},
        "configs": results,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, cfg)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
