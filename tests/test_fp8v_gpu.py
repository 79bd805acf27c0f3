"""GPU parity of the float8 e5m2 V path (the reference's fp8_v branch,
flash_attention_forward.py:208-211, 217, 453-456, 466) against the oracle:
known answers that pin the e5m2 rounding of P and the unrounded row sum, the
provable per-element bound for random inputs, strided V and the split mode."""
import numpy as np
import pytest
import torch

from ascend_rsfa import flash_attention_forward as faf
from oracle import attention as A

pytestmark = pytest.mark.gpu


def _run(q, k, v8, causal, scale, **kw):
    print(f"fp8v: shape={tuple(q.shape)} causal={causal} scale={scale} {kw}", flush=True)
    o = faf.forward(q.cuda(), k.cuda(), v8.cuda(), causal, scale, **kw)
    torch.cuda.synchronize()
    return o.float().cpu()


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_two_key_case_rounds_p_and_sums_it_unrounded(d, causal):
    q = torch.zeros(1, 1, 2, d)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 2, d)
    k[0, 0, 1, 0] = float(np.log(0.6))
    v = torch.zeros(1, 1, 2, d)
    v[0, 0, 1] = 1.0
    q, k, v8 = q.half(), k.half(), v.to(torch.float8_e5m2)
    p1 = float(np.exp(float(k[0, 0, 1, 0])))
    o = _run(q, k, v8, causal, 1.0)
    want = 0.625 / (1.0 + p1)  # e5m2(0.6) = 0.625 over the unrounded sum 1.6
    assert abs(o[0, 0, 1, 0].item() - want) < 1e-3
    assert abs(o[0, 0, 1, 0].item() - 0.625 / 1.625) > 3e-3  # not the rounded sum
    assert abs(o[0, 0, 0, 0].item() - (0.0 if causal else want)) < 1e-3


@pytest.mark.parametrize("causal", [False, True])
def test_zero_scale_gives_the_mean_of_v(causal):
    q, k, v = A.make_inputs(2, 3, 200, 64, seed=5)
    v8 = v.to(torch.float8_e5m2)
    o = _run(q, k, v8, causal, 0.0)
    ref = A.reference_attention_fp8v(q, k, v8, causal, 0.0)
    assert (o - ref).abs().max().item() < 2e-3


CASES = [  # Z, H, N, D, causal, sm_scale
    (2, 4, 300, 64, False, 0.125),
    (1, 4, 512, 128, True, 0.08),
    (2, 2, 256, 256, False, 0.0625),
    (1, 2, 1000, 128, True, 0.5),
    (2, 2, 333, 32, True, 0.2),
    (1, 3, 130, 16, False, 0.25),
    (1, 8, 2048, 128, False, 1 / np.sqrt(128)),
]


@pytest.mark.parametrize("case", CASES)
def test_random_inputs_within_the_rounding_bound(case):
    Z, H, N, D, causal, scale = case
    q, k, v = A.make_inputs(Z, H, N, D, seed=N + D)
    v8 = v.to(torch.float8_e5m2)
    o = _run(q, k, v8, causal, scale)
    heads = [(0, 0), (Z - 1, H - 1)]
    exact = A.reference_attention(q, k, v8.float(), causal, scale, heads=heads)
    bound = A.fp8v_error_bound(q, k, v8, causal, scale, heads=heads)
    got = torch.stack([o[z, h] for z, h in heads])
    assert torch.isfinite(got).all()
    excess = ((got - exact).abs() - bound).max().item()
    assert excess <= 0, f"outside the bound by {excess}"


def test_p_rounding_is_active():
    q, k, v = A.make_inputs(1, 2, 512, 64, seed=9)
    v8 = v.to(torch.float8_e5m2)
    o8 = _run(q, k, v8, False, 0.05)
    o16 = _run(q, k, v8.half(), False, 0.05)  # same V values, P rounded to fp16 instead
    assert (o8 - o16).abs().max().item() > 1e-3


def test_strided_float8_v_matches_contiguous():
    q, k, v = A.make_inputs(2, 3, 160, 64, seed=13)
    store = v.permute(0, 2, 1, 3).contiguous().to(torch.float8_e5m2)  # [Z, N, H, D] storage
    v_view = store.permute(0, 2, 1, 3)  # [Z, H, N, D] view, strides (N*H*D, D, H*D, 1)
    assert not v_view.is_contiguous() and all(s % 16 == 0 for s in v_view.stride()[:3])
    a = _run(q, k, v_view.cuda(), True, 0.3)
    b = _run(q, k, v_view.contiguous(), True, 0.3)
    assert torch.equal(a, b)


@pytest.mark.parametrize("D", [64, 128, 32, 16])
def test_split_mode_with_float8_v(D):
    """The two-launch causal split with a float8 V on the byte path (the split
    state alone in the workspace)."""
    q, k, v = A.make_inputs(1, 4, 700, D, seed=17)
    v8 = v.to(torch.float8_e5m2)
    o = _run(q, k, v8, True, 0.25, split=True)
    heads = [(0, 0), (0, 3)]
    exact = A.reference_attention(q, k, v8.float(), True, 0.25, heads=heads)
    bound = A.fp8v_error_bound(q, k, v8, True, 0.25, heads=heads)
    got = torch.stack([o[z, h] for z, h in heads])
    assert ((got - exact).abs() <= bound).all()


def test_reference_entry_point_accepts_float8_v():
    q, k, v = A.make_inputs(1, 2, 256, 64, seed=21)
    v8 = v.to(torch.float8_e5m2)
    print("fp8v: attention() entry point", flush=True)
    o = faf.attention(q.cuda(), k.cuda(), v8.cuda(), False, 0.125, *faf.get_tiling(1, 2, 256, 64, False))
    torch.cuda.synchronize()
    assert o.dtype == torch.float16 and o.shape == q.shape
    exact = A.reference_attention(q, k, v8.float(), False, 0.125)
    bound = A.fp8v_error_bound(q, k, v8, False, 0.125)
    assert ((o.float().cpu() - exact).abs() <= bound).all()


def _raw_args(q, k, v, o, dtype_code, causal=False, flags=0, ws=0, ws_bytes=0):
    import ctypes

    from ascend_rsfa import _native

    a = _native.FwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype = dtype_code
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    a.z, a.h, a.n_ctx, a.head_dim = q.shape
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", o)):
        getattr(a, name)[:] = list(t.stride())
    a.sm_scale, a.causal, a.flags = 0.1, int(causal), flags
    a.workspace, a.workspace_bytes = ws, ws_bytes
    return a


def test_workspace_size_and_alignment_are_checked_before_any_launch():
    import ctypes

    from ascend_rsfa import _native

    lib = _native.lib()
    # a float8 V needs no workspace at any head dim; the causal split needs its state
    q, k, v = (t.cuda() for t in A.make_inputs(1, 2, 128, 32, seed=23))
    v8, o = v.to(torch.float8_e5m2), torch.empty_like(q)
    assert all(lib.rsfa_v8_workspace_bytes(1, 2, 128, d) == 0 for d in (16, 32, 64, 128, 256))
    run = lambda a: lib.rsfa_attention_fwd(ctypes.byref(a), None)  # noqa: E731
    print("workspace checks", flush=True)
    assert run(_raw_args(q, k, v8, o, _native.DTYPE_F16_V8E5M2)) == _native.OK
    split = int(lib.rsfa_split_workspace_bytes(1, 2, 128, 32, 128))
    ws = torch.empty(split // 4 + 16, dtype=torch.float32, device="cuda")
    for vv, code in ((q, _native.DTYPE_F16), (v8, _native.DTYPE_F16_V8E5M2)):
        a = _raw_args(q, k, vv, o, code, causal=True, flags=_native.FLAG_CAUSAL_SPLIT)
        a.block_m, a.block_n = 128, 64
        assert run(a) == _native.E_WORKSPACE
        a.workspace, a.workspace_bytes = ws.data_ptr(), split - 4
        assert run(a) == _native.E_WORKSPACE
        a.workspace, a.workspace_bytes = ws.data_ptr() + 2, split
        assert run(a) == _native.E_ALIGN
        a.workspace, a.workspace_bytes = ws.data_ptr(), split
        assert run(a) == _native.OK
    msg = lib.rsfa_strerror(_native.E_WORKSPACE).decode()
    assert "rsfa_split_workspace_bytes" in msg
    torch.cuda.synchronize()


@pytest.mark.parametrize("N", [64, 1024])
def test_uncompiled_tile_request_within_the_rounding_bound(N):
    """A (256, 32) tile request with a float8 V at head dim 128, a tile no
    head-dim-128 kernel has: the nearest compiled byte-V tile runs."""
    Z, H, D = 1, 4, 128
    q, k, v = A.make_inputs(Z, H, N, D, seed=N + 3)
    v8 = v.to(torch.float8_e5m2)
    o = _run(q, k, v8, False, 0.1, BM=256, BN=32, exact_tile=True)
    heads = [(0, 0), (0, H - 1)]
    exact = A.reference_attention(q, k, v8.float(), False, 0.1, heads=heads)
    bound = A.fp8v_error_bound(q, k, v8, False, 0.1, heads=heads)
    got = torch.stack([o[z, h] for z, h in heads])
    assert torch.isfinite(got).all()
    excess = ((got - exact).abs() - bound).max().item()
    assert excess <= 0, f"outside the bound by {excess}"


@pytest.mark.parametrize("D,tile", [(128, (256, 64)), (128, (256, 128)), (128, (128, 64)),
                                    (64, (256, 128)), (64, (128, 64))])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N,scale", [(1024, 0.1), (777, -0.3)])
def test_byte_v_tiles_within_the_rounding_bound(D, tile, causal, N, scale):
    """A float8 V's bytes go into LDS and P.V runs on the e5m2 MFMA: at head
    dims 64 and 128 every compiled tile (D=128: ping-pong
    (256, 64), (256, 128), the 4-wave (128, 64); D=64: ping-pong (256, 128),
    4-wave (128, 64)), whole and ragged key tiles, a negative scale, more tasks
    than workgroups, against the exact result within the per-element bound of
    the e5m2 rounding of P."""
    Z, H = 2, 24
    q, k, v = A.make_inputs(Z, H, N, D, seed=N + tile[1] + int(causal) + D)
    v8 = v.to(torch.float8_e5m2)
    o = _run(q, k, v8, causal, scale, BM=tile[0], BN=tile[1], exact_tile=True)
    heads = [(0, 0), (0, 7), (1, 13), (Z - 1, H - 1)]
    exact = A.reference_attention(q, k, v8.float(), causal, scale, heads=heads)
    bound = A.fp8v_error_bound(q, k, v8, causal, scale, heads=heads)
    got = torch.stack([o[z, h] for z, h in heads])
    assert torch.isfinite(got).all()
    excess = ((got - exact).abs() - bound).max().item()
    assert excess <= 0, f"outside the bound by {excess}"


def test_strided_byte_v_matches_contiguous():
    """A float8 V read as bytes through its strides ([Z, N, H, D] storage)."""
    q, k, v = A.make_inputs(2, 3, 700, 128, seed=31)
    store = v.permute(0, 2, 1, 3).contiguous().to(torch.float8_e5m2)
    v_view = store.permute(0, 2, 1, 3)
    assert not v_view.is_contiguous()
    a = _run(q, k, v_view.cuda(), True, 0.3)
    b = _run(q, k, v_view.contiguous(), True, 0.3)
    assert torch.equal(a, b)


@pytest.mark.parametrize("N", [1, 17, 100])
@pytest.mark.parametrize("causal", [False, True])
def test_byte_v_short_sequences(N, causal):
    """Head dim 128 float8 V with fewer keys than one tile: the partial-tile
    loads (rows past the sequence re-read its last row) and the masked P.V
    (sub-tiles no row sees are not read) of the byte path."""
    q, k, v = A.make_inputs(2, 3, N, 128, seed=40 + N)
    v8 = v.to(torch.float8_e5m2)
    o = _run(q, k, v8, causal, 0.2)
    heads = [(0, 0), (1, 2)]
    exact = A.reference_attention(q, k, v8.float(), causal, 0.2, heads=heads)
    bound = A.fp8v_error_bound(q, k, v8, causal, 0.2, heads=heads)
    got = torch.stack([o[z, h] for z, h in heads])
    assert torch.isfinite(got).all()
    excess = ((got - exact).abs() - bound).max().item()
    assert excess <= 0, f"outside the bound by {excess}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_float8_v_lse_is_the_exact_logsumexp(D, causal):
    """With a float8 V the row sums add the unrounded P (as the reference's
    fp8_v branch), so the LSE output is the logsumexp of the scaled scores,
    independent of V's rounding: the oracle's exact LSE to 1e-3."""
    q, k, v = A.make_inputs(2, 3, 333, D, seed=50 + D)
    v8 = v.to(torch.float8_e5m2)
    print(f"fp8v lse: D={D} causal={causal}", flush=True)
    o, lse = faf.forward(q.cuda(), k.cuda(), v8.cuda(), causal, 0.3, return_lse=True)
    torch.cuda.synchronize()
    heads = [(0, 1), (1, 2)]
    _, ref_lse = A.reference_attention(q, k, v.float(), causal, 0.3, return_lse=True, heads=heads)
    got = torch.stack([lse[z, h].cpu() for z, h in heads])
    assert torch.isfinite(got).all()
    assert (got - ref_lse).abs().max().item() < 1e-3


def _byte_tiles(D, causal):
    """The compiled tiles a float8 V can run at head dim D (each reached by
    the request nearest to it)."""
    reqs = [(256, 128), (256, 64), (256, 32), (128, 64), (128, 32)]
    return sorted({tuple(faf.resolve_tiling(D, causal, bm, bn)) for bm, bn in reqs if not (causal and bn > bm)})


def _peaked_inputs(N, D, causal, seed):
    """Query i attends to key pi(i) alone: K rows are distinct random +-1
    rows, Q[i] = K[pi(i)], so the score of pi(i) is D while every other key
    scores at most D - 2; sm_scale (1 from D = 64 on, 16 below, returned) puts
    every other visible key at least 30 log2 units below (checked here in
    float64): every other P is below 2^-30 of P[pi(i)] = 1.  V rows are
    distinct e5m2 values, so O[i] = V[pi(i)] exactly names the key the kernel
    paired with row i.  Non-causal pi is a permutation (every key position of
    every 64-key MFMA group and tile once); causal pi(i) in [i - 63, i]."""
    g = torch.Generator().manual_seed(seed)
    scale = 1.0 if D >= 64 else 16.0
    k = (torch.randint(0, 2, (N, D), generator=g) * 2 - 1).float()
    for _ in range(64):  # re-draw repeated rows (likely at D = 16)
        _, inv, cnt = torch.unique(k, dim=0, return_inverse=True, return_counts=True)
        rep_rows = torch.nonzero(torch.tensor([bool(cnt[inv[i]] > 1) and bool((inv[:i] == inv[i]).any())
                                               for i in range(N)])).flatten()
        if rep_rows.numel() == 0:
            break
        k[rep_rows] = (torch.randint(0, 2, (rep_rows.numel(), D), generator=g) * 2 - 1).float()
    if causal:
        pi = torch.tensor([i - int(torch.randint(0, min(i, 63) + 1, (1,), generator=g)) for i in range(N)])
    else:
        pi = torch.randperm(N, generator=g)
    q = k[pi]
    s = (q.double() @ k.double().T)
    if causal:
        s.masked_fill_(A.causal_mask(N), float("-inf"))
    top = s.gather(1, pi[:, None]).squeeze(1)
    others = s.scatter(1, pi[:, None], float("-inf")).max(dim=1).values
    assert bool((top == D).all()) and bool(((top - others) * scale * 1.4426950408889634 >= 30).all()), \
        "construction: a row's peak is not 30 log2 units above its other keys"
    v8 = torch.from_numpy(A.round_e5m2((torch.randn(N, D, generator=g) * 2).numpy())).to(torch.float8_e5m2)
    assert len({tuple(r) for r in v8.view(torch.uint8).tolist()}) == N, "V rows must be distinct"
    return q.half()[None, None], k.half()[None, None], v8[None, None], pi, scale


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N", [64, 273, 1024])
def test_peaked_rows_return_their_key_value_on_every_tile(D, causal, N):
    """Known answers for the float8 V P.V path on every compiled tile of
    every head dim: V's bytes in LDS (byte-transposing reads, 16-byte chunks
    swizzled from 64-byte rows on, 32-byte rows with the D = 16 filler chunk),
    P and V paired byte by byte inside each 64-key MFMA.  A key read from the
    wrong row, chunk, lane or 16-key group gives another row's V."""
    q, k, v8, pi, scale = _peaked_inputs(N, D, causal, seed=1000 + N + D + causal)
    want = v8[0, 0].float()[pi]
    for tile in _byte_tiles(D, causal):
        o = _run(q, k, v8, causal, scale, BM=tile[0], BN=tile[1])[0, 0]
        bad = (o - want).abs() > 2.0 ** -10 * want.abs()
        assert not bool(bad.any()), (f"tile {tile}: {int(bad.any(dim=1).sum())} of {N} rows differ from "
                                     f"V[pi(i)], first row {int(bad.any(dim=1).nonzero()[0])}")


def _first_key_max_inputs(Z, H, N, D, seed):
    """Inputs whose kernel P is exactly the oracle's: key 0 carries every
    row's largest score, so the running max is the exact row max from the
    first key tile on (no lagging max), and every score is a multiple of 1/8
    (Q in {0, +-1/2}, K in {0, +-1/4}: exact in fp16 and in fp32 sums), so
    with sm_scale = ln 2 each P = 2^(-j/8).  Those values lie at least 1.7 %
    from every rounding midpoint of e5m2, so the kernel's exp2 and the
    oracle's float64 exp round them alike.  Coordinate 0 is reserved: Q[:, 0]
    = 1, K[j, 0] = 0 for j > 0, K[0, 0] = B, the smallest multiple of 1/4
    that puts key 0 at least 1/8 above each row's other keys.  One P value is
    an e5m2 tie, 2^-17 (half the smallest subnormal): draws where a score
    sits exactly 17 below its row max are skipped (the next draw of the
    seed's sequence is taken).  V ~ N(0, 1) rounded to e5m2."""
    g = torch.Generator().manual_seed(seed)
    for _ in range(64):
        q = (torch.randint(-1, 2, (Z, H, N, D), generator=g) * 0.5).float()
        k = (torch.randint(-1, 2, (Z, H, N, D), generator=g) * 0.25).float()
        q[..., 0] = 1.0
        k[..., 0] = 0.0
        s = q.double() @ k.double().transpose(-1, -2)
        need = (s[..., 1:].max(dim=-1).values - s[..., 0]).max().item() + 0.125
        k[:, :, 0, 0] = float(np.ceil(max(need, 0.0) * 4) / 4)
        s = q.double() @ k.double().transpose(-1, -2)
        if not bool((s - s[..., :1] == -17.0).any()):
            break
    else:
        raise AssertionError("construction: no draw without an e5m2 tie")
    v8 = torch.from_numpy(A.round_e5m2(torch.randn(Z, H, N, D, generator=g).numpy())).to(torch.float8_e5m2)
    return q.half(), k.half(), v8


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N", [200, 1000])
def test_exact_row_max_matches_the_rounded_p_oracle(D, causal, N):
    """With the row max on key 0 and scores on a 1/8 grid the kernel rounds
    exactly the P the oracle rounds (reference_attention_fp8v: P = 2^(-j/8),
    1 -> 1, 0.917 -> 0.875, ...), so O must match it to fp16 rounding, not
    just within the loose per-element rounding bound: on every byte tile of
    every head dim, at lengths whose last 64-key group is partial."""
    Z, H = 1, 2
    q, k, v8 = _first_key_max_inputs(Z, H, N, D, seed=2000 + N + D)
    scale = float(np.log(2.0))
    heads = [(0, 0), (0, H - 1)]
    want = A.reference_attention_fp8v(q, k, v8, causal, scale, heads=heads)
    for tile in _byte_tiles(D, causal):
        o = _run(q, k, v8, causal, scale, BM=tile[0], BN=tile[1])
        got = torch.stack([o[z, h] for z, h in heads])
        excess = ((got - want).abs() - (1e-4 + 2.0 ** -10 * want.abs())).max().item()
        assert excess <= 0, f"tile {tile}: outside fp16 rounding of the exact-P oracle by {excess:.3e}"
