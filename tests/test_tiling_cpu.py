"""CPU tests of the measured tiling search (ascend_rsfa.tiling): candidate
rules (reference tiling/search_optimal_tiling.py:47-81), the correctness gate
the reference's search lacks, the reference's result layout, and the tiling
cache behind get_tiling.  The search runs here with a CPU attention function
(the closed form, or a copy of it that corrupts chosen tilings), so the gate
is exercised without a GPU."""
import json

import pytest
import torch

from ascend_rsfa import flash_attention_forward as faf
from ascend_rsfa import tiling


@pytest.mark.parametrize("n", [64, 1024, 4096, 8192])
@pytest.mark.parametrize("causal", [False, True])
def test_request_candidates_follow_the_reference_rules(n, causal):
    got = tiling.request_candidates(n, 128, causal)
    assert got, n
    for bm, bn in got:
        assert bm in (32, 64, 128, 256) and bm <= n
        assert bn in (32, 64, 128, 256, 512) and bn <= n
        assert bn != 512 or n >= 4096
        assert bm * bn <= 65536
        assert not (causal and bn > bm)  # the NaN-giving causal requests are never tried
    assert len(set(got)) == len(got)
    assert got == sorted(got, key=lambda x: (x[0] * x[1], x[0], x[1]))
    if n >= 4096 and not causal:
        assert (128, 512) in got


@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_compiled_candidates_partition_the_requests(d, causal):
    reqs = tiling.request_candidates(2048, d, causal)
    cands = tiling.compiled_candidates(2048, d, causal)
    assert cands
    seen = [r for rs in cands.values() for r in rs]
    assert sorted(seen) == sorted(reqs)  # every request runs exactly one instantiation
    for run in cands:
        assert faf.resolve_tiling(d, causal, run[0], run[1]) == run  # a compiled shape maps to itself


def test_sample_heads_cover_first_and_last():
    assert tiling.sample_heads(128, 8) == [(0, 0), (127, 7)]
    assert tiling.sample_heads(1, 1) == [(0, 0)]
    hs = tiling.sample_heads(4, 4, count=4)
    assert hs[0] == (0, 0) and hs[-1] == (3, 3) and len(hs) == 4


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g)


def test_closed_form_matches_float64_brute_force():
    q, k, v = (_rand((2, 2, 9, 16), s) for s in (1, 2, 3))
    heads = [(0, 1), (1, 0)]
    for causal in (False, True):
        ref = tiling.closed_form(q, k, v, causal, 0.3, heads)
        for i, (z, h) in enumerate(heads):
            s = (q[z, h].double() @ k[z, h].double().T) * 0.3
            if causal:
                s = s + torch.triu(torch.full((9, 9), float("-inf"), dtype=torch.float64), 1)
            want = torch.softmax(s, -1) @ v[z, h].double()
            assert torch.allclose(ref[i].double(), want, atol=1e-5)
        if causal:  # row 0 sees key 0 only
            assert torch.allclose(ref[:, 0], torch.stack([v[z, h, 0] for z, h in heads]), atol=1e-6)


def test_gate_accepts_close_and_rejects_far_or_nonfinite():
    q, k, v = (_rand((1, 2, 16, 8), s) for s in (4, 5, 6))
    heads = [(0, 0), (0, 1)]
    ref = tiling.closed_form(q, k, v, False, 0.5, heads)
    o = torch.zeros(1, 2, 16, 8)
    o[0, 0], o[0, 1] = ref[0], ref[1]
    ok, err, why = tiling.gate(o + 1e-3, ref, heads)
    assert ok and err < 2e-3 and why == ""
    bad = o.clone()
    bad[0, 1, 3, 2] += 0.5
    ok, err, why = tiling.gate(bad, ref, heads)
    assert not ok and err == pytest.approx(0.5, abs=1e-6) and "outside" in why
    nan = o.clone()
    nan[0, 0, 0, 0] = float("nan")
    ok, _, why = tiling.gate(nan, ref, heads)
    assert not ok and "non-finite" in why


def _cpu_attention(corrupt=()):
    """The closed form on every head; tilings in ``corrupt`` get NaN (0) or a shifted row (1)."""
    def fn(q, k, v, causal, sm_scale, bm, bn):
        Z, H = q.shape[:2]
        o = tiling.closed_form(q, k, v, causal, sm_scale, [(z, h) for z in range(Z) for h in range(H)])
        o = o.reshape(q.shape).to(q.dtype)
        for i, t in enumerate(corrupt):
            if (bm, bn) == t:
                if i % 2 == 0:
                    o[0, 0, 1, 1] = float("nan")
                else:
                    o[-1, -1, 5] += 1.0
        return o
    return fn


def test_search_gates_out_wrong_tilings_and_keeps_the_reference_layout():
    cands = {(64, 32): [(64, 32)], (128, 64): [(128, 64), (64, 64)], (256, 64): [(256, 64)]}
    rec = tiling.search_case(2, 2, 64, 16, True, torch.float32, 0.5, warmup=0, iters=1,
                             attention_fn=_cpu_attention(corrupt=[(64, 32), (256, 64)]), device="cpu",
                             candidates=cands)
    assert set(rec) >= {"params", "best", "top3", "all_tested", "failed_count", "gate"}
    assert rec["failed_count"] == 2
    rejected = {(r["BM"], r["BN"]) for r in rec["failed"]}
    assert rejected == {(64, 32), (256, 64)}
    assert all(r["error"].startswith("correctness gate") for r in rec["failed"])
    assert (rec["best"]["BM"], rec["best"]["BN"]) == (128, 64)
    assert rec["best"]["requests"] == [[128, 64], [64, 64]]
    assert [r["avg_ms"] for r in rec["all_tested"]] == sorted(r["avg_ms"] for r in rec["all_tested"])
    json.dumps(rec)  # serialisable as the reference's results are


def test_search_with_every_tiling_wrong_has_no_best():
    cands = {(64, 32): [(64, 32)], (128, 64): [(128, 64)]}
    rec = tiling.search_case(1, 1, 32, 16, False, torch.float32, 0.5, warmup=0, iters=1,
                             attention_fn=_cpu_attention(corrupt=[(64, 32), (128, 64)]), device="cpu",
                             candidates=cands)
    assert rec["best"] is None and rec["top3"] == [] and rec["failed_count"] == 2


def test_search_records_exceptions_as_failures():
    def fn(q, k, v, causal, sm_scale, bm, bn):
        if bm == 256:
            raise ValueError("no such tile")
        return _cpu_attention()(q, k, v, causal, sm_scale, bm, bn)
    rec = tiling.search_case(1, 1, 32, 16, False, torch.float32, 0.5, warmup=0, iters=1, attention_fn=fn,
                             device="cpu", candidates={(256, 64): [(256, 64)], (128, 64): [(128, 64)]})
    assert rec["failed"][0]["error"].startswith("ValueError")
    assert (rec["best"]["BM"], rec["best"]["BN"]) == (128, 64)


def test_cache_round_trip_and_results(tmp_path):
    c = tiling.TilingCache(device_name="test")
    c.put(32, 8, 2048, 128, False, torch.float16, 256, 64)
    assert c.lookup(32, 8, 2048, 128, False) == (256, 64)
    assert c.lookup(32, 8, 2048, 128, True) is None
    assert c.lookup(32, 8, 2048, 128, False, torch.bfloat16) is None
    rec = {"C9": {"params": {"Z": 2, "H": 4, "N_CTX": 512, "HEAD_DIM": 64, "causal": True,
                             "dtype": "torch.float16"}, "best": {"BM": 128, "BN": 64}},
           "C10": {"params": {"Z": 1, "H": 1, "N_CTX": 64, "HEAD_DIM": 64, "causal": False,
                              "dtype": "torch.float16"}, "best": None}}
    c.add_results(rec)
    assert c.lookup(2, 4, 512, 64, True) == (128, 64)
    assert c.lookup(1, 1, 64, 64, False) is None
    p = tmp_path / "cache.json"
    c.save(p)
    d = tiling.TilingCache.load(p)
    assert d.entries == c.entries and d.device_name == "test"
    p.write_text(json.dumps({"entries": {"1,1,1,64,0,float16": [128]}}))
    with pytest.raises(ValueError):
        tiling.TilingCache.load(p)


def test_get_tiling_answers_from_an_active_cache(tmp_path):
    model = faf.get_tiling(32, 8, 2048, 128, False)
    other = (128, 64) if model != (128, 64) else (256, 128)
    c = tiling.TilingCache()
    c.put(32, 8, 2048, 128, False, torch.float16, *other)
    c.put(32, 8, 2048, 64, False, torch.float16, 96, 48)  # not a compiled shape: ignored
    try:
        tiling.use_cache(c)
        assert faf.get_tiling(32, 8, 2048, 128, False) == other
        assert faf.get_tiling(32, 8, 2048, 64, False) == faf_model(32, 8, 2048, 64, False)
        assert faf.get_tiling(32, 8, 1024, 128, False) == faf_model(32, 8, 1024, 128, False)
        p = tmp_path / "c.json"
        c.save(p)
        tiling.use_cache(str(p))
        assert faf.get_tiling(32, 8, 2048, 128, False) == other
    finally:
        tiling.use_cache(None)
    assert faf.get_tiling(32, 8, 2048, 128, False) == model


def faf_model(Z, H, N, D, causal):
    """get_tiling without a cache (the library's cost model)."""
    saved = tiling.active_cache()
    try:
        tiling.use_cache(None)
        return faf.get_tiling(Z, H, N, D, causal)
    finally:
        tiling.use_cache(saved)


def test_reference_tilings_cover_the_reference_cases_and_are_valid_requests():
    # the tiles of the reference's get_tiling table for its 12 cases
    # (flash_attention_forward.py:652-663), as the comparison runs them
    assert sorted(tiling.REFERENCE_TILINGS) == [c[0] for c in tiling.REFERENCE_CASES]
    for idx, Z, H, N, D, causal, dtype in tiling.REFERENCE_CASES:
        bm, bn = tiling.REFERENCE_TILINGS[idx]
        assert (bm, bn) == ((64 if D == 256 else 128), 64) if causal else bn >= 256
        rbm, rbn = faf.resolve_tiling(D, causal, bm, bn)
        assert rbm >= 64 and rbn >= 32 and (rbn <= rbm or not causal)
