"""Pins of the oracle's restatement of the reference's fp8_v branch
(flash_attention_forward.py:208-211, 217): e5m2 rounding of P for P.V, row sums
of the unrounded P.  CPU only."""
import numpy as np
import pytest
import torch

from oracle import attention as A


def test_round_e5m2_matches_torch_across_binades_ties_and_subnormals():
    rs = np.random.RandomState(0)
    x = np.concatenate([rs.randn(20000).astype(np.float32) * s for s in (1e-6, 1e-4, 1e-2, 1.0, 100.0, 5000.0)])
    # exact ties between neighbouring e5m2 values (round to even) and the subnormal edge
    ties = np.array([1.125, 1.375, 1.625, 1.875, 2.25, 0.5625, 3 * 2.0 ** -17, 2.0 ** -17, 2.0 ** -15 * 1.125],
                    dtype=np.float32)
    x = np.concatenate([x, ties, -ties])
    got = A.round_e5m2(x)
    want = torch.from_numpy(x).to(torch.float8_e5m2).float().numpy()
    assert np.array_equal(got, want)


def test_every_finite_e5m2_value_is_fixed():
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e5m2).float().numpy()
    fin = np.isfinite(codes)
    assert fin.sum() == 256 - 8  # +-inf and six NaN codes (exponent all ones)
    assert np.array_equal(A.round_e5m2(codes[fin]), codes[fin])
    assert A.round_e5m2(np.float32(A.E5M2_MAX)) == A.E5M2_MAX


def _kat_two_keys(n_extra=0):
    """Query rows see key 0 with p = 1 and key 1 with p = 0.6 (rounds to 0.625 in e5m2)."""
    D = 16
    q = torch.zeros(1, 1, 2 + n_extra, D)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 2 + n_extra, D)
    k[0, 0, 1, 0] = float(np.log(0.6))
    if n_extra:
        k[0, 0, 2:, 0] = -30.0  # negligible extra keys
    v = torch.zeros(1, 1, 2 + n_extra, D)
    v[0, 0, 1] = 1.0
    return q.half(), k.half(), v.to(torch.float8_e5m2)


def test_two_key_case_pins_the_unrounded_row_sum():
    q, k, v8 = _kat_two_keys()
    p1 = float(np.exp(float(k[0, 0, 1, 0])))  # the fp16 score gives p = 0.6001
    assert A.round_e5m2(np.float32(p1)) == 0.625
    o = A.reference_attention_fp8v(q, k, v8, False, 1.0)
    want = 0.625 / (1.0 + p1)
    assert abs(float(o[0, 0, 0, 0]) - want) < 1e-6
    # a planted mistake: summing the rounded P would give 0.625 / 1.625
    assert abs(0.625 / 1.625 - want) > 5e-3


def test_zero_scale_gives_the_mean_of_v():
    q, k, v = A.make_inputs(1, 2, 37, 32, seed=3)
    v8 = v.to(torch.float8_e5m2)
    o = A.reference_attention_fp8v(q, k, v8, False, 0.0)
    assert torch.allclose(o, v8.float().mean(dim=2, keepdim=True).expand_as(o), atol=1e-6)
    oc = A.reference_attention_fp8v(q, k, v8, True, 0.0)
    pref = torch.cumsum(v8.float(), dim=2) / torch.arange(1, 38).view(1, 1, 37, 1)
    assert torch.allclose(oc, pref, atol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [0.05, 0.5])
def test_bound_holds_for_the_oracles_own_rounding_and_is_not_vacuous(causal, scale):
    q, k, v = A.make_inputs(2, 2, 64, 32, seed=11)
    v8 = v.to(torch.float8_e5m2)
    exact = A.reference_attention(q, k, v8.float(), causal, scale)
    o8 = A.reference_attention_fp8v(q, k, v8, causal, scale)
    b = A.fp8v_error_bound(q, k, v8, causal, scale)
    assert ((o8 - exact).abs() <= b).all()
    assert (o8 - exact).abs().max() > 1e-4  # P rounding shows
    assert b.max() < 0.2 * v8.float().abs().max()  # and the bound is a real constraint
    # a planted mistake the bound catches: the key order of V reversed
    wrong = A.reference_attention_fp8v(q, k, v8.float().flip(2).to(torch.float8_e5m2), causal, scale)
    assert ((wrong - exact).abs() > b).any()
