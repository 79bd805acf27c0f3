"""The operator file loaded by path, the way every reference harness loads it.

The reference's harnesses (benchmarks/run_correctness_test.py:58-65,
run_final_benchmark.py:73-81, tiling/search_optimal_tiling.py:84-91) import
``flash_attention_forward.py`` with ``importlib.util.spec_from_file_location``
under a bare module name (no package) and then use ``attention`` and
``get_tiling``.  The CPU test does that in a fresh interpreter whose
``sys.path`` does not hold this package; the GPU test runs the path-loaded
``attention`` against the oracle.
"""
import importlib.util
import json
import os
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNEL = os.path.join(ROOT, "ascend-rsfa_amd", "ascend_rsfa", "flash_attention_forward.py")


def load_by_path(path):
    """Module from a file path under a name made from the file name, registered
    in sys.modules before it runs (the reference harnesses' recipe)."""
    name = os.path.splitext(os.path.basename(path))[0]
    for ch in " -()":
        name = name.replace(ch, "_" if ch in " -" else "")
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


_CHILD = f"""
import importlib.util, json, os, sys
# this package must not be importable from the start: the module finds it itself
sys.path = [p for p in sys.path if 'ascend-rsfa_amd' not in p and p not in ('', {ROOT!r})]
def load_by_path(path):
    name = os.path.splitext(os.path.basename(path))[0].replace('-', '_')
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod
mod = load_by_path(sys.argv[1])
assert mod.__name__ == 'flash_attention_forward' and not mod.__package__
assert callable(mod.attention) and callable(mod.get_tiling)
print(json.dumps([mod.get_tiling(128, 8, 2048, 128, True), mod.get_tiling(128, 8, 2048, 128, False)]))
"""

def test_loads_by_file_path_without_the_package_on_sys_path(tmp_path):
    env = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    proc = subprocess.run([sys.executable, "-c", _CHILD, KERNEL], cwd=tmp_path, env=env,
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-3000:]
    tilings = json.loads(proc.stdout.strip().splitlines()[-1])
    for bm, bn in tilings:
        assert bm in (64, 128, 256) and bn in (32, 64, 128)


@pytest.mark.gpu
def test_path_loaded_attention_matches_the_oracle():
    from oracle import attention as A

    mod = load_by_path(KERNEL)
    Z, H, N, D = 2, 3, 384, 128
    q, k, v = A.make_inputs(Z, H, N, D, seed=77, std=0.5)
    for causal in (True, False):
        BM, BN = mod.get_tiling(Z, H, N, D, causal)
        print(f"path-loaded attention causal={causal} tiling={BM}x{BN}", flush=True)
        out = mod.attention(q.cuda(), k.cuda(), v.cuda(), causal, 0.5, BM, BN)
        torch.cuda.synchronize()
        ref = A.reference_attention(q, k, v, causal, 0.5)
        assert torch.allclose(out.float().cpu(), ref, atol=1e-2, rtol=1e-2)


@pytest.mark.gpu
def test_get_num_compute_cores_is_the_device_cu_count():
    mod = load_by_path(KERNEL)
    n = mod.get_num_compute_cores()
    assert n == torch.cuda.get_device_properties(0).multi_processor_count
    print(f"compute units: {n}", flush=True)
