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


def test_inputs_follow_the_fingerprinted_recipe():
    import torch

    c1 = next(c for c in bench.CONFIGS if c[0] == "C1")
    q, k, v = bench.make_inputs(torch, c1)
    assert q.dtype == k.dtype == v.dtype == torch.float16 and q.device.type == "cpu"
    assert bench.fingerprint_check(torch, "C1", (q, k, v)) is True
    # another draw does not match
    assert bench.fingerprint_check(torch, "C1", (k, q, v)) is False


def test_headline_is_the_north_star_shape_and_c3_is_beside_it():
    name, B, H, S, D, causal, scale, seed = bench.CONFIGS[0][:8]
    assert (name, B, H, S, D, causal) == ("target-noncausal", 128, 8, 2048, 128, False) == (bench.HEADLINE,) + (
        128, 8, 2048, 128, False)
    assert abs(scale - 128 ** -0.5) < 1e-12
    c3 = next(c for c in bench.CONFIGS if c[0] == bench.CAUSAL_TARGET)
    assert c3[1:7] == (128, 8, 2048, 128, True, 0.5)


def test_cpu_baseline_reports_cores_and_model():
    import torch

    cfg = ("tiny", 1, 2, 128, 64, True, 0.5, 7)
    inputs = bench.make_inputs(torch, cfg)
    before = torch.get_num_threads()
    try:
        cb = bench.cpu_baseline(torch, cfg, inputs, budget_s=0.2)
    finally:
        torch.set_num_threads(before)
    assert cb["kind"] == "port" and cb["unit"] == "TFLOP/s" and cb["value"] > 0
    assert cb["cores"] == bench.host_threads() >= 1 and cb["os_cpu_count"] == os.cpu_count()
    assert isinstance(cb["cpu_model"], str) and cb["cpu_model"]


def test_roofline_bound_is_the_larger_floor():
    by_name = {c[0]: c for c in bench.CONFIGS}
    # C4-causal (64,8,1024,256): 2.75e11 FLOP at 2.5 PFLOP/s = 0.110 ms, below its
    # 1.07 GB at 8 TB/s = 0.134 ms: HBM-bound, reported in GB/s
    c4c = by_name["C4-causal"]
    rf = bench.roofline(c4c, {"ms_per_call": 0.268})
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == bench.PEAK_HBM_GBS
    assert abs(rf["achieved"] - bench.algo_bytes(64, 8, 1024, 256, True) / 0.268e-3 / 1e9) < 0.1
    assert abs(rf["frac"] - rf["achieved"] / bench.PEAK_HBM_GBS) < 1e-4
    # the target (1024 FLOP/B) is MFMA-bound, in TFLOP/s
    rt = bench.roofline(by_name["target-noncausal"], {"ms_per_call": 2.0})
    assert rt["bound"] == "mfma" and rt["unit"] == "TFLOP/s"
    assert abs(rt["achieved"] - bench.flops(128, 8, 2048, 128, False) / 2.0e-3 / 1e12) < 0.1
    # a traffic figure names the committed profile it comes from
    if rt["traffic"] is not None:
        assert "not measured in this run" in rt["traffic_source"]


def test_median_window_is_reported():
    """time_config times --windows windows of exactly --steps calls and reports
    the median one (a fake clock stands in for the HIP events)."""
    import types
    windows_ms = iter([12.0, 30.0, 10.0])  # elapsed ms of 3 windows of 10 steps

    class Event:
        def __init__(self, enable_timing=False):
            pass

        def record(self, stream=None):
            pass

        def elapsed_time(self, other):
            return next(windows_ms)

    calls = []
    cuda = types.SimpleNamespace(Event=Event, synchronize=lambda: None, current_stream=lambda: None)
    fake_torch = types.SimpleNamespace(cuda=cuda)
    fake_F = types.SimpleNamespace(get_tiling=lambda *a: (256, 64), attention=lambda *a: calls.append(1))
    cfg = bench.CONFIGS[0]
    res = bench.time_config(fake_F, fake_torch, cfg, (None, None, None), True, steps=10, warmup=2, windows=3)
    assert len(calls) == 2 + 3 * 10
    assert res["windows_ms"] == [1.2, 3.0, 1.0] and res["ms_per_call"] == 1.2


class _FakeSmi:
    """Stands in for the amd-smi child process: communicate() returns its JSON."""

    def __init__(self, text):
        self.text = text

    def communicate(self, timeout=None):
        return self.text, ""

    def kill(self):
        pass


def _smi_json(n_gpus, power=1400, clocks=(1578, 1553, 1582, 1543, 1580, 1549, 1580, 1549)):
    gpu = {"gpu": 0, "power": {"socket_power": {"value": power, "unit": "W"}, "gfx_voltage": "N/A"},
           "clock": {**{f"gfx_{i}": {"clk": {"value": c, "unit": "MHz"}, "min_clk": "N/A"}
                        for i, c in enumerate(clocks)},
                     "mem_0": {"clk": {"value": 2000, "unit": "MHz"}}, "fclk_0": "N/A"}}
    return json.dumps({"gpu_data": [gpu] * n_gpus})


def test_power_reading_parses_socket_power_and_gfx_clocks():
    r = bench.smi_result(_FakeSmi(_smi_json(1)))
    assert r == {"socket_power_w": 1400, "gfx_mhz_min": 1543, "gfx_mhz_max": 1582, "gfx_mhz_mean": 1564.2}
    # not attributable (several GPUs), not parseable, or no tool: no reading
    assert bench.smi_result(_FakeSmi(_smi_json(2))) is None
    assert bench.smi_result(_FakeSmi("amd-smi: error")) is None
    assert bench.smi_result(None) is None
