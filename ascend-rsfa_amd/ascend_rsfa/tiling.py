"""Measured tiling search and tiling cache, with a correctness gate.

Counterpart of the reference's tiling/search_optimal_tiling.py (and of the
checks in check_optimal_tiling.py / retest_optimal_tiling.py).  The reference
times every (BM, BN) candidate of its 12 shapes and keeps the fastest
(search_optimal_tiling.py:95-143) without looking at the results: its causal
D=256 winner (64, 256) is a tiling that gives NaN there
(tiling_search_optimized.json, case_02; benchmarks/run_correctness_test.py:24-25).

Here:

* the candidates are the compiled gfx950 tile shapes that valid requests
  resolve to: the request rules of search_optimal_tiling.py:47-81 (powers of
  two up to N_CTX, BM * BN <= 65536, BN = 512 from N_CTX >= 4096 on), plus
  BN <= BM for causal calls, mapped through ``resolve_tiling``; requests that
  run the same instantiation are timed once.  The reference's BM <= 128 for
  D >= 256 (an Ascend register budget, 70-72) is left out: it would hide the
  256-row D=256 tile gfx950 runs;
* each candidate's output on the timed inputs is compared with the fp32 closed
  form softmax(Q K^T * scale) V on sampled heads (atol = rtol = 1e-2, no
  non-finite values); a candidate that fails the gate is reported and never
  becomes ``best``;
* results keep the reference's JSON layout per case (``params``, ``best``,
  ``top3``, ``all_tested``, ``failed_count``) and add the gate's outcome;
* a ``TilingCache`` holds gated winners by shape; ``get_tiling`` of
  ``flash_attention_forward`` answers from the active cache (``use_cache``,
  or the path in ``RSFA_TILING_CACHE``) before falling back to the library's
  cost model.

Command line::

    python -m ascend_rsfa.tiling --cases baseline --output tiling.json \
        [--cache cache.json] [--warmup 5] [--iters 20]
    python -m ascend_rsfa.tiling --reference-tilings [--output rows.json]
"""
import argparse
import json
import os
import sys
import time

import torch

# (idx, Z, H, N_CTX, HEAD_DIM, causal, dtype): the reference's 12 search cases
# (search_optimal_tiling.py:33-46).
REFERENCE_CASES = [
    (1, 128, 8, 1024, 128, True, torch.float16),
    (2, 128, 8, 1024, 256, True, torch.float16),
    (3, 128, 8, 2048, 128, True, torch.float16),
    (4, 128, 8, 2048, 256, True, torch.float16),
    (5, 128, 8, 4096, 128, True, torch.float16),
    (6, 128, 8, 8192, 64, True, torch.float16),
    (7, 128, 8, 1024, 128, False, torch.float16),
    (8, 128, 8, 1024, 256, False, torch.float16),
    (9, 128, 8, 2048, 128, False, torch.float16),
    (10, 128, 8, 2048, 256, False, torch.float16),
    (11, 128, 8, 4096, 128, False, torch.float16),
    (12, 128, 8, 8192, 64, False, torch.float16),
]

# The benchmark configurations of this build (C1-C5, and the B=128 non-causal
# shape of the performance target).
BASELINE_CASES = [
    ("C1", 2, 8, 1024, 128, True, torch.float16),
    ("C2", 32, 8, 2048, 128, False, torch.float16),
    ("C3", 128, 8, 2048, 128, True, torch.float16),
    ("C4n", 64, 8, 1024, 256, False, torch.float16),
    ("C4c", 64, 8, 1024, 256, True, torch.float16),
    ("C5", 4, 16, 8192, 64, True, torch.float16),
    ("T", 128, 8, 2048, 128, False, torch.float16),
]

GATE_ATOL = 1e-2
GATE_RTOL = 1e-2


def request_candidates(N_CTX, HEAD_DIM, causal):
    """(BM, BN) requests a search tries, by the reference's rules
    (search_optimal_tiling.py:47-81, the branch for kernels that take any BM),
    without the causal BN > BM requests that give NaN in the reference.
    HEAD_DIM is accepted for the reference's signature; no rule here uses it."""
    bms = [b for b in (32, 64, 128, 256) if b <= N_CTX]
    bns = [b for b in (32, 64, 128, 256) if b <= N_CTX]
    if N_CTX >= 4096:
        bns.append(512)
    out = [(bm, bn) for bm in bms for bn in bns if bm * bn <= 65536 and not (causal and bn > bm)]
    out.sort(key=lambda x: (x[0] * x[1], x[0], x[1]))
    return out


def compiled_candidates(N_CTX, HEAD_DIM, causal, dtype=torch.float16):
    """Distinct compiled instantiations the requests resolve to:
    ``{(BM, BN) run: [requests]}``, in request order."""
    from .flash_attention_forward import resolve_tiling
    out = {}
    for req in request_candidates(N_CTX, HEAD_DIM, causal):
        try:
            got = resolve_tiling(HEAD_DIM, causal, req[0], req[1], dtype)
        except ValueError:
            continue
        out.setdefault(tuple(got), []).append(req)
    return out


def sample_heads(Z, H, count=2):
    """(z, h) heads the gate checks: the first, the last and count - 2 evenly
    spaced between them."""
    n = Z * H
    idx = sorted({0, n - 1} | {i * n // max(1, count - 1) for i in range(1, max(1, count - 1))})
    return [(i // H, i % H) for i in idx]


def closed_form(q, k, v, causal, sm_scale, heads):
    """fp32 softmax(Q K^T * scale) V for the listed (z, h) heads: [len(heads), N, D]."""
    outs = []
    for z, h in heads:
        qf, kf, vf = q[z, h].float(), k[z, h].float(), v[z, h].float()
        s = (qf @ kf.transpose(0, 1).contiguous()) * sm_scale
        if causal:
            n = s.shape[0]
            s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool, device=s.device), 1), float("-inf"))
        outs.append(torch.softmax(s, dim=-1) @ vf)
    return torch.stack(outs)


def gate(o, ref, heads, atol=GATE_ATOL, rtol=GATE_RTOL):
    """Check the sampled heads of ``o`` against ``ref``: returns (ok, max_abs_err, reason)."""
    got = torch.stack([o[z, h].float() for z, h in heads])
    if not torch.isfinite(got).all():
        return False, float("nan"), "non-finite output"
    err = (got - ref).abs()
    max_err = float(err.max())
    bad = err > atol + rtol * ref.abs()
    if bad.any():
        return False, max_err, f"{int(bad.sum())} elements outside atol={atol} rtol={rtol}"
    return True, max_err, ""


def _timer_ms(fn, warmup, iters, device):
    if device.type == "cuda":
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize(device)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize(device)
        return e0.elapsed_time(e1) / iters
    for _ in range(warmup):
        fn()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    return (time.perf_counter() - t0) * 1e3 / iters


def make_inputs(Z, H, N_CTX, HEAD_DIM, dtype, device, seed=42, std=0.5):
    """Q, K, V ~ N(0, std^2) as in the reference's search (search_optimal_tiling.py:102-106)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    shape = (Z, H, N_CTX, HEAD_DIM)
    return [(torch.randn(shape, generator=g) * std).to(dtype).to(device) for _ in range(3)]


def search_case(Z, H, N_CTX, HEAD_DIM, causal, dtype=torch.float16, sm_scale=0.5, warmup=3, iters=10,
                attention_fn=None, device=None, heads=None, candidates=None, verbose=False):
    """Time and gate every candidate tiling of one shape.

    ``attention_fn(q, k, v, causal, sm_scale, BM, BN)`` defaults to this
    package's ``forward`` with ``exact_tile=True``; ``candidates`` defaults to ``compiled_candidates``.
    Returns the case record (reference layout plus ``gate``)."""
    if attention_fn is None:
        from .flash_attention_forward import forward

        def attention_fn(q, k, v, causal, sm_scale, bm, bn):
            # each candidate runs its own instantiation, whatever RSFA_TILE_HINT says
            return forward(q, k, v, causal, sm_scale, bm, bn, exact_tile=True)
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    if candidates is None:
        candidates = compiled_candidates(N_CTX, HEAD_DIM, causal, dtype)
    q, k, v = make_inputs(Z, H, N_CTX, HEAD_DIM, dtype, device)
    heads = heads or sample_heads(Z, H)
    ref = closed_form(q, k, v, causal, sm_scale, heads)
    tested, failed = [], []
    for (bm, bn), reqs in candidates.items():
        rec = {"BM": bm, "BN": bn, "requests": [list(r) for r in reqs]}
        try:
            o = attention_fn(q, k, v, causal, sm_scale, bm, bn)
            if device.type == "cuda":
                torch.cuda.synchronize(device)
            ok, err, why = gate(o, ref, heads)
            rec["max_abs_err"] = err
            if not ok:
                rec["error"] = "correctness gate: " + why
                failed.append(rec)
                if verbose:
                    print(f"    BM={bm:3d}, BN={bn:3d} -> REJECTED ({why}, max err {err:.3g})")
                continue
            rec["avg_ms"] = round(_timer_ms(lambda: attention_fn(q, k, v, causal, sm_scale, bm, bn),
                                            warmup, iters, device), 4)
        except (RuntimeError, ValueError, AssertionError) as e:
            rec["error"] = f"{type(e).__name__}: {e}"
            failed.append(rec)
            if verbose:
                print(f"    BM={bm:3d}, BN={bn:3d} -> FAILED ({rec['error']})")
            continue
        tested.append(rec)
        if verbose:
            print(f"    BM={bm:3d}, BN={bn:3d} -> {rec['avg_ms']:10.4f} ms (max err {rec['max_abs_err']:.3g})")
    tested.sort(key=lambda r: r["avg_ms"])
    flops = 4.0 * Z * H * N_CTX * N_CTX * HEAD_DIM * (0.5 if causal else 1.0)
    for r in tested:
        r["tflops"] = round(flops / (r["avg_ms"] * 1e-3) / 1e12, 1)
    return {
        "params": {"Z": Z, "H": H, "N_CTX": N_CTX, "HEAD_DIM": HEAD_DIM, "causal": bool(causal),
                   "dtype": str(dtype), "sm_scale": sm_scale},
        "best": tested[0] if tested else None,
        "top3": tested[:3],
        "all_tested": tested,
        "failed": failed,
        "failed_count": len(failed),
        "gate": {"heads": [list(h) for h in heads], "atol": GATE_ATOL, "rtol": GATE_RTOL,
                 "reference": "fp32 softmax(QK^T*scale)V"},
    }


# The tiles a reference user passes for its 12 cases: the reference's own
# get_tiling table (flash_attention_forward.py:652-663).
REFERENCE_TILINGS = {1: (128, 64), 2: (64, 64), 3: (128, 64), 4: (64, 64), 5: (128, 64), 6: (128, 64),
                     7: (128, 256), 8: (64, 256), 9: (128, 256), 10: (64, 256), 11: (128, 256), 12: (128, 512)}


def compare_reference_tilings(warmup=2, iters=5, sm_scale=0.5, rounds=6, verbose=False):
    """The reference's 12 cases timed three ways on this GPU.

    * ``ours``: ``attention(..., *get_tiling(...))``, this build's choice;
    * ``ref_hint``: ``forward(..., BM, BN, tile_hint=True)`` with the
      reference's tile for the case: the request is only checked and the tile
      of ``get_tiling`` runs (hint mode, ``RSFA_TILE_HINT=1``);
    * ``ref_exact``: ``attention(..., BM, BN)``, the call a reference user
      makes: the compiled tile nearest to the reference's request.

    Inputs: Q, K, V ~ N(0, 0.5^2) in fp16 drawn on the GPU (seed 7 + case),
    sm_scale 0.5, as the reference's benchmark harness uses
    (benchmarks/run_correctness_test.py:119-126).  Each time is the median of
    ``rounds`` interleaved rounds of ``iters`` calls.  Returns one record per
    case.
    """
    from .flash_attention_forward import attention, forward, get_tiling, resolve_tiling

    device = torch.device("cuda", torch.cuda.current_device())
    rows = []
    for idx, Z, H, N, D, causal, dtype in REFERENCE_CASES:
        g = torch.Generator(device=device)
        g.manual_seed(7 + idx)
        q, k, v = (torch.randn((Z, H, N, D), generator=g, device=device).mul_(0.5).to(dtype) for _ in range(3))
        ref_tile = REFERENCE_TILINGS[idx]
        ours = tuple(get_tiling(Z, H, N, D, causal, dtype))
        exact = tuple(resolve_tiling(D, causal, *ref_tile, dtype=dtype))
        runs = {
            "ours": lambda: attention(q, k, v, causal, sm_scale, *ours),
            "ref_hint": lambda: forward(q, k, v, causal, sm_scale, *ref_tile, tile_hint=True),
            "ref_exact": lambda: forward(q, k, v, causal, sm_scale, *ref_tile, exact_tile=True),
        }
        fl = 4.0 * Z * H * N * N * D * (0.5 if causal else 1.0)
        rec = {"case": idx, "Z": Z, "H": H, "N_CTX": N, "HEAD_DIM": D, "causal": causal,
               "ref_tile": list(ref_tile), "ours_tile": list(ours), "ref_exact_tile": list(exact)}
        for name, fn in runs.items():
            o = fn()
            torch.cuda.synchronize(device)
            if not bool(torch.isfinite(o).all()):
                raise RuntimeError(f"case {idx}: {name} gave non-finite output")
        # about a second of launches first (the clocks settle under load), then
        # the three runs interleaved, the order reversed every round; medians
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 1.0:
            for fn in runs.values():
                fn()
            torch.cuda.synchronize(device)
        times = {name: [] for name in runs}
        order = list(runs)
        for r in range(rounds):
            for name in (order if r % 2 == 0 else order[::-1]):
                times[name].append(_timer_ms(runs[name], warmup, iters, device))
        for name in runs:
            ms = sorted(times[name])[len(times[name]) // 2]
            rec[name + "_ms"] = round(ms, 4)
            rec[name + "_tflops"] = round(fl / (ms * 1e-3) / 1e12, 1)
        rec["ref_exact_vs_ours"] = round(rec["ref_exact_ms"] / rec["ours_ms"], 3)
        rec["ref_hint_vs_ours"] = round(rec["ref_hint_ms"] / rec["ours_ms"], 3)
        rows.append(rec)
        if verbose:
            print(f"case {idx:02d} Z={Z} H={H} N={N} D={D} {'causal' if causal else 'non-causal'}: "
                  f"ours {ours} {rec['ours_ms']:.3f} ms | ref hint {ref_tile} {rec['ref_hint_ms']:.3f} ms | "
                  f"ref exact {exact} {rec['ref_exact_ms']:.3f} ms", flush=True)
        del q, k, v
        torch.cuda.empty_cache()
    return rows


def _key(Z, H, N_CTX, HEAD_DIM, causal, dtype):
    return f"{int(Z)},{int(H)},{int(N_CTX)},{int(HEAD_DIM)},{int(bool(causal))},{str(dtype).replace('torch.', '')}"


class TilingCache:
    """Gated search winners by exact shape: ``{key: [BM, BN]}`` in a JSON file."""

    def __init__(self, entries=None, device_name=""):
        self.entries = dict(entries or {})
        self.device_name = device_name

    def lookup(self, Z, H, N_CTX, HEAD_DIM, causal, dtype=torch.float16):
        hit = self.entries.get(_key(Z, H, N_CTX, HEAD_DIM, causal, dtype))
        return tuple(hit) if hit else None

    def put(self, Z, H, N_CTX, HEAD_DIM, causal, dtype, bm, bn):
        self.entries[_key(Z, H, N_CTX, HEAD_DIM, causal, dtype)] = [int(bm), int(bn)]

    def add_results(self, results):
        """Enter the gated best of every case record of a search."""
        for rec in results.values():
            b, p = rec.get("best"), rec["params"]
            if b:
                dt = getattr(torch, p["dtype"].replace("torch.", ""))
                self.put(p["Z"], p["H"], p["N_CTX"], p["HEAD_DIM"], p["causal"], dt, b["BM"], b["BN"])

    def save(self, path):
        with open(path, "w") as f:
            json.dump({"device": self.device_name, "entries": self.entries}, f, indent=1, sort_keys=True)

    @classmethod
    def load(cls, path):
        with open(path) as f:
            d = json.load(f)
        ent = d.get("entries", {})
        for k, v in ent.items():
            if not (isinstance(v, list) and len(v) == 2 and all(isinstance(x, int) for x in v)):
                raise ValueError(f"tiling cache {path}: bad entry {k!r}: {v!r}")
        return cls(ent, d.get("device", ""))


_active = None
_env_checked = False


def use_cache(cache):
    """Make ``cache`` (a TilingCache, a path, or None to disable) the one
    ``get_tiling`` consults."""
    global _active, _env_checked
    _env_checked = True
    _active = TilingCache.load(cache) if isinstance(cache, (str, os.PathLike)) else cache


def active_cache():
    """The cache ``get_tiling`` consults (first use reads ``RSFA_TILING_CACHE``)."""
    global _active, _env_checked
    if not _env_checked:
        _env_checked = True
        path = os.environ.get("RSFA_TILING_CACHE")
        if path:
            _active = TilingCache.load(path)
    return _active


def main(argv=None):
    ap = argparse.ArgumentParser(description="Measured (BM, BN) search with a correctness gate")
    ap.add_argument("--cases", choices=["baseline", "reference", "all"], default="baseline")
    ap.add_argument("--output", default=None, help="JSON file for the full results")
    ap.add_argument("--cache", default=None, help="JSON tiling cache to create or extend with the winners")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--sm-scale", type=float, default=0.5)
    ap.add_argument("--reference-tilings", action="store_true",
                    help="time the reference's 12 cases with the reference's tiles against get_tiling's")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("the search times the GPU kernels: no GPU visible", file=sys.stderr)
        return 2
    if args.reference_tilings:
        rows = compare_reference_tilings(args.warmup, args.iters, args.sm_scale, verbose=True)
        if args.output:
            with open(args.output, "w") as f:
                json.dump(rows, f, indent=1)
        return 0
    cases = []
    if args.cases in ("baseline", "all"):
        cases += list(BASELINE_CASES)
    if args.cases in ("reference", "all"):
        cases += [(f"case_{c[0]:02d}",) + tuple(c[1:]) for c in REFERENCE_CASES]
    results = {}
    for name, Z, H, N, D, causal, dtype in cases:
        print(f"[{name}] Z={Z} H={H} N_CTX={N} D={D} {'causal' if causal else 'non-causal'}", flush=True)
        rec = search_case(Z, H, N, D, causal, dtype, args.sm_scale, args.warmup, args.iters, verbose=True)
        results[name] = rec
        b = rec["best"]
        print(f"  => BEST: " + (f"BM={b['BM']}, BN={b['BN']}, {b['avg_ms']} ms, {b['tflops']} TFLOP/s"
                                if b else "none passed the gate"), flush=True)
    if args.output:
        with open(args.output, "w") as f:
            json.dump(results, f, indent=1)
    if args.cache:
        cache = TilingCache.load(args.cache) if os.path.exists(args.cache) else TilingCache(
            device_name=torch.cuda.get_device_name())
        cache.add_results(results)
        cache.save(args.cache)
    return 0 if all(r["best"] for r in results.values()) else 1


if __name__ == "__main__":
    sys.exit(main())
