"""The reference's own case list at full size (tiling/search_optimal_tiling.py
case list, the twelve Z=128, H=8 shapes its correctness and benchmark harnesses
run), with the reference harness's input distribution: Q, K, V ~ N(0, 0.5^2)
and sm_scale = 0.5 (benchmarks/run_correctness_test.py:119-126).  Every output
must be finite; the first and last heads are checked against the fp32 oracle at
atol = rtol = 1e-2, the repository's own tolerance.  The reference published
max |err| <= 9.77e-4 for these cases on its NPU (correctness_test_results.txt:
15-33); this build's errors are printed next to it."""
import pytest
import torch

from ascend_rsfa import flash_attention_forward as faf
from ascend_rsfa import tiling
from oracle import attention as A

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", tiling.REFERENCE_CASES, ids=lambda c: f"case_{c[0]:02d}")
def test_reference_case_full_size(case):
    idx, Z, H, N, D, causal, dtype = case
    print(f"reference case {idx:02d}: Z={Z} H={H} N={N} D={D} causal={causal}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(100 + idx)
    q, k, v = (torch.randn((Z, H, N, D), generator=g, device="cuda").mul_(0.5).to(dtype) for _ in range(3))
    o = faf.attention(q, k, v, causal, 0.5, *faf.get_tiling(Z, H, N, D, causal))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all())
    heads = [(0, 0), (Z - 1, H - 1)]
    ref = A.reference_attention(q, k, v, causal, 0.5, heads=heads)
    got = torch.stack([o[z, h] for z, h in heads]).float().cpu()
    err = (got - ref).abs().max().item()
    print(f"  max |err| {err:.3e}", flush=True)
    assert torch.allclose(got, ref, atol=1e-2, rtol=1e-2), f"max |err| {err:.3e}"
