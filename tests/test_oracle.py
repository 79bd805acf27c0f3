"""Pins the oracle (CPU only).

The reference ships no tensors and its golden op (torch_npu.npu_fusion_attention)
needs an Ascend NPU, so the oracle is pinned by independent computations and by
mathematics: float64 brute-force fixtures, torch's SDPA in float64, closed
forms, invariants, and planted mistakes that each of these must catch.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as A

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_golden.npz")


def _fixture_cases():
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files})
    return data, names


def _as_bhnd(a, dtype=torch.float16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype)[None, None]


def _run_case(fn, data, name):
    meta = data[name + "/meta"]
    causal, scale = bool(meta[2]), float(meta[3])
    q, k, v = (_as_bhnd(data[name + "/" + t]) for t in "qkv")
    o, lse = fn(q, k, v, causal, scale)
    return o[0, 0].double().numpy(), lse[0, 0].double().numpy(), data[name + "/o"], data[name + "/lse"]


def _oracle(q, k, v, causal, scale):
    return A.reference_attention(q, k, v, causal, scale, return_lse=True)


def test_oracle_matches_golden_fixtures():
    data, names = _fixture_cases()
    assert len(names) >= 12
    for name in names:
        o, lse, o_ref, lse_ref = _run_case(_oracle, data, name)
        assert np.abs(o - o_ref).max() < 1e-5, name
        assert np.abs(lse - lse_ref).max() < 2e-5, name


def test_onehot_fixture_retrieves_rows():
    data, _ = _fixture_cases()
    perm = data["onehot_n16/perm"]
    v = data["onehot_n16/v"].astype(np.float64)
    o_ref = data["onehot_n16/o"]
    # query i only matches key perm[i]; with scale 64 the other weights are e^-64
    assert np.abs(o_ref - v[perm]).max() < 1e-12


def test_brute_force_helper_matches_fixtures():
    data, names = _fixture_cases()
    for name in names[:4]:
        meta = data[name + "/meta"]
        o, lse = A.brute_force_attention_f64(data[name + "/q"], data[name + "/k"], data[name + "/v"],
                                             bool(meta[2]), float(meta[3]))
        assert np.abs(o - data[name + "/o"]).max() < 1e-12


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 3, 64, 32), (1, 2, 97, 64), (1, 1, 130, 128)])
def test_oracle_matches_sdpa_float64(causal, shape):
    q, k, v = A.make_inputs(*shape, seed=3)
    scale = 0.37
    ref = torch.nn.functional.scaled_dot_product_attention(q.double(), k.double(), v.double(), is_causal=causal,
                                                           scale=scale)
    out = A.reference_attention(q, k, v, causal, scale)
    assert (out.double() - ref).abs().max().item() < 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_zero_scale_gives_mean_of_visible_values(causal):
    q, k, v = A.make_inputs(1, 2, 50, 16, seed=4)
    out = A.reference_attention(q, k, v, causal, 0.0)
    vf = v.float()
    if causal:
        expect = torch.cumsum(vf, dim=2) / torch.arange(1, 51, dtype=torch.float32)[:, None]
    else:
        expect = vf.mean(dim=2, keepdim=True).expand_as(vf)
    assert (out - expect).abs().max().item() < 1e-5


def test_causal_first_row_is_first_value():
    q, k, v = A.make_inputs(2, 2, 33, 64, seed=5)
    out = A.reference_attention(q, k, v, True, 0.9)
    assert torch.equal(out[:, :, 0, :], v[:, :, 0, :].float())


def test_joint_key_value_permutation_invariance():
    q, k, v = A.make_inputs(1, 2, 40, 32, seed=6)
    perm = torch.randperm(40, generator=torch.Generator().manual_seed(0))
    a = A.reference_attention(q, k, v, False, 0.5)
    b = A.reference_attention(q, k[:, :, perm], v[:, :, perm], False, 0.5)
    assert (a - b).abs().max().item() < 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_output_is_convex_combination(causal):
    q, k, v = A.make_inputs(1, 3, 64, 16, seed=7)
    out = A.reference_attention(q, k, v, causal, 1.3)
    vmin = v.float().amin(dim=2, keepdim=True)
    vmax = v.float().amax(dim=2, keepdim=True)
    assert bool((out >= vmin - 1e-5).all()) and bool((out <= vmax + 1e-5).all())


# --- planted mistakes: each mutant must fail at least one pinning check -------

def _mut_shifted_diagonal(q, k, v, causal, scale):
    Z, H, N, D = q.shape
    s = q.float() @ k.float().transpose(-1, -2) * scale
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(N, N, dtype=torch.bool), diagonal=0), float("-inf"))
        s[..., 0, 0] = 0.0  # keep row 0 finite
    return torch.softmax(s, -1) @ v.float(), torch.logsumexp(s, -1)


def _mut_dropped_scale(q, k, v, causal, scale):
    return A.reference_attention(q, k, v, causal, 1.0, return_lse=True)


def _mut_transposed_v(q, k, v, causal, scale):
    o, lse = A.reference_attention(q, k, v.transpose(-1, -2).contiguous(), causal, scale, return_lse=True)
    return o, lse


def _mut_wrong_axis(q, k, v, causal, scale):
    s = q.float() @ k.float().transpose(-1, -2) * scale
    if causal:
        s = s.masked_fill(A.causal_mask(q.shape[2]), float("-inf"))
    p = torch.softmax(s, -2)
    return torch.nan_to_num(p) @ v.float(), torch.logsumexp(s, -1)


@pytest.mark.parametrize("mutant", [_mut_shifted_diagonal, _mut_dropped_scale, _mut_transposed_v, _mut_wrong_axis])
def test_planted_mistake_is_caught(mutant):
    data, names = _fixture_cases()
    caught = False
    for name in names:
        meta = data[name + "/meta"]
        if mutant is _mut_transposed_v and meta[0] != meta[1]:
            continue  # needs a square head to run at all
        try:
            o, lse, o_ref, lse_ref = _run_case(mutant, data, name)
        except RuntimeError:
            caught = True
            break
        if not np.isfinite(o).all() or np.abs(o - o_ref).max() > 1e-2:
            caught = True
            break
    assert caught, mutant.__name__


# --- the C restatement of the reference's tiled algorithm ----------------------

@pytest.mark.parametrize("case", [
    (1, 2, 64, 64, False, 64, 16),     # small kernel path (N <= 128)
    (1, 2, 64, 64, True, 64, 16),      # small causal path (N <= 64)
    (1, 2, 256, 64, False, 64, 32),    # tiled non-causal
    (1, 2, 256, 64, True, 64, 32),     # causal prefix/diagonal split
    (1, 1, 256, 128, True, 128, 64),
    (1, 1, 256, 256, False, 64, 64),
])
def test_blockwise_restatement_matches_closed_form(case):
    Z, H, N, D, causal, BM, BN = case
    q, k, v = A.make_inputs(Z, H, N, D, seed=9, std=0.5)
    ref = A.reference_attention(q, k, v, causal, 0.5)
    out = A.blockwise_attention(q, k, v, causal, 0.5, BM, BN)
    err = (out.float() - ref).abs().max().item()
    assert torch.allclose(out.float(), ref, atol=1e-2, rtol=1e-2)
    # the reference reports max |err| <= 9.77e-4 for this input distribution
    # (benchmarks/correctness_test_results.txt:15-33)
    assert err <= 2 * 9.765625e-4, err


def test_blockwise_rejects_shapes_the_reference_cannot_run():
    q, k, v = A.make_inputs(1, 1, 200, 64, seed=1)
    with pytest.raises(ValueError):
        A.blockwise_attention(q, k, v, False, 0.5, 64, 64)
    q, k, v = A.make_inputs(1, 1, 256, 64, seed=1)
    with pytest.raises(ValueError):
        A.blockwise_attention(q, k, v, True, 0.5, 64, 128)


def test_blockwise_lse_matches_closed_form():
    q, k, v = A.make_inputs(1, 2, 256, 64, seed=10)
    _, lse_ref = A.reference_attention(q, k, v, False, 0.5, return_lse=True)
    _, lse = A.blockwise_attention(q, k, v, False, 0.5, 64, 64, return_lse=True)
    assert (lse - lse_ref).abs().max().item() < 1e-4


def test_c_half_conversions_match_numpy():
    lib = A.c_library()
    all_halves = np.arange(65536, dtype=np.uint16)
    ref = all_halves.view(np.float16).astype(np.float32)
    got = np.array([lib.rsfa_oracle_f16_to_f32(int(h)) for h in all_halves[::7]], dtype=np.float32)
    r = ref[::7]
    finite = np.isfinite(r)
    assert np.array_equal(got[finite], r[finite])
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(3000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 300, 7e4)])
    with np.errstate(over="ignore"):  # the 7e4 scale overflows to inf on purpose
        want = xs.astype(np.float16).view(np.uint16)
    got16 = np.array([lib.rsfa_oracle_f32_to_f16(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got16, want)
    bf = np.array([lib.rsfa_oracle_f32_to_bf16(float(x)) for x in xs[:2000]], dtype=np.uint16)
    want_bf = torch.from_numpy(xs[:2000]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, want_bf)


def _fingerprints():
    import json
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "input_fingerprints.json")
    with open(path) as f:
        return json.load(f)["configs"]


def test_input_fingerprints_cover_the_baseline_configs_and_match_c1():
    fp = _fingerprints()
    assert sorted(fp) == ["C1", "C2", "C3", "C4", "C5", "target-noncausal"]
    c1 = fp["C1"]
    q, k, v = A.make_inputs(*c1["shape"], c1["seed"])
    assert A.fingerprint(q, k, v) == c1["sha256"]
    # a different seed, or k and v drawn in the other order, changes it
    q2, k2, v2 = A.make_inputs(*c1["shape"], c1["seed"] + 1)
    assert A.fingerprint(q2, k2, v2) != c1["sha256"]
    assert A.fingerprint(q, v, k) != c1["sha256"]


@pytest.mark.parametrize("dtype,p1r", [(torch.float16, 0.60009765625), (torch.bfloat16, 0.6015625)])
def test_rounded_p_lse_known_answer(dtype, p1r):
    # two keys whose scores differ by ln(0.6): P = (1, 0.6) unrounded, (1, 0.6 rounded) as the kernels sum it
    d = 16
    q = torch.zeros(1, 1, 2, d)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 2, d)
    k[0, 0, 1, 0] = 1.0
    scale = math.log(0.6)  # s = (0, ln 0.6) for both query rows
    assert torch.equal(q.to(dtype).float(), q) and torch.equal(k.to(dtype).float(), k)
    lse_r = A.reference_lse_rounded_p(q.to(dtype), k.to(dtype), False, scale)
    assert abs(lse_r[0, 0, 0].item() - math.log(1.0 + p1r)) < 1e-7
    _, lse_u = A.reference_attention(q.to(dtype), k.to(dtype), k.to(dtype), False, scale, return_lse=True)
    assert abs(lse_u[0, 0, 0].item() - math.log(1.6)) < 1e-6
    # the two normalisations differ by more than the tests' LSE tolerance
    assert abs(math.log(1.0 + p1r) - math.log(1.6)) > 5e-5


@pytest.mark.parametrize("dtype,rel", [(torch.float16, 2.0 ** -11), (torch.bfloat16, 2.0 ** -8)])
def test_rounded_p_lse_within_one_rounding_of_the_reference(dtype, rel):
    q, k, v = A.make_inputs(1, 2, 96, 32, seed=12, dtype=dtype)
    for causal in (False, True):
        lse_r = A.reference_lse_rounded_p(q, k, causal, 0.4)
        _, lse_u = A.reference_attention(q, k, v, causal, 0.4, return_lse=True)
        diff = (lse_r - lse_u.double()).abs().max().item()
        assert diff <= rel * 1.01 + 1e-6, diff
        assert diff > 0.0
