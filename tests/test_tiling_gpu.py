"""GPU tests of the measured tiling search: every compiled tiling of a shape
passes the correctness gate, a tiling whose output is corrupted on the host is
gated out and cannot win, and the winners drive get_tiling through the cache."""
import pytest
import torch

from ascend_rsfa import flash_attention_forward as faf
from ascend_rsfa import tiling

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,causal", [(128, False), (128, True), (64, True), (256, False)])
def test_every_compiled_tiling_passes_the_gate(d, causal):
    print(f"search Z=2 H=4 N=512 D={d} causal={causal}", flush=True)
    rec = tiling.search_case(2, 4, 512, d, causal, torch.float16, 0.5, warmup=1, iters=2)
    cands = tiling.compiled_candidates(512, d, causal)
    assert rec["failed_count"] == 0, rec["failed"]
    assert len(rec["all_tested"]) == len(cands)
    assert (rec["best"]["BM"], rec["best"]["BN"]) in cands
    for r in rec["all_tested"]:
        assert r["max_abs_err"] < 1e-2 and r["avg_ms"] > 0 and r["tflops"] > 0


def test_a_corrupted_tiling_is_rejected_and_cannot_win():
    cands = tiling.compiled_candidates(512, 128, False)
    assert len(cands) >= 2
    bad = sorted(cands)[0]

    def fn(q, k, v, causal, sm_scale, bm, bn):
        o = faf.forward(q, k, v, causal, sm_scale, bm, bn, exact_tile=True)
        if (bm, bn) == bad:
            o = o.clone()
            o[0, 0, 7, 3] = float("nan")
        return o

    print(f"search with tiling {bad} corrupted", flush=True)
    rec = tiling.search_case(2, 4, 512, 128, False, torch.float16, 0.5, warmup=1, iters=2, attention_fn=fn)
    assert [(r["BM"], r["BN"]) for r in rec["failed"]] == [bad]
    assert (rec["best"]["BM"], rec["best"]["BN"]) != bad


def test_search_winner_drives_get_tiling():
    print("search Z=2 H=8 N=1024 D=128 causal, then get_tiling from the cache", flush=True)
    rec = tiling.search_case(2, 8, 1024, 128, True, torch.float16, 0.5, warmup=1, iters=3)
    cache = tiling.TilingCache(device_name=torch.cuda.get_device_name())
    cache.add_results({"x": rec})
    best = (rec["best"]["BM"], rec["best"]["BN"])
    try:
        tiling.use_cache(cache)
        assert faf.get_tiling(2, 8, 1024, 128, True) == best
        q, k, v = tiling.make_inputs(2, 8, 1024, 128, torch.float16, "cuda")
        o = faf.attention(q, k, v, True, 0.5, *faf.get_tiling(2, 8, 1024, 128, True))
        ref = tiling.closed_form(q, k, v, True, 0.5, [(1, 7)])
        assert (o[1, 7].float() - ref[0]).abs().max().item() < 1e-2
    finally:
        tiling.use_cache(None)
