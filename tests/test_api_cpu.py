"""CPU tests of the Python surface (ascend_rsfa.flash_attention_forward).

The checks mirror the reference module's behaviour that does not need a
device: its assertions (flash_attention_forward.py:553-554), get_tiling's
contract (624-665) and the names a harness loads (attention, get_tiling).
"""
import importlib

import pytest
import torch

from ascend_rsfa import flash_attention_forward as F


def test_reference_names_present():
    mod = importlib.import_module("ascend_rsfa.flash_attention_forward")
    for name in ("attention", "get_tiling", "get_num_compute_cores", "_attention"):
        assert hasattr(mod, name)
    assert mod.attention == mod._attention.apply
    assert issubclass(mod._attention, torch.autograd.Function)


def test_head_dim_mismatch_asserts_like_reference():
    q = torch.zeros(1, 1, 64, 64, dtype=torch.float16)
    k = torch.zeros(1, 1, 64, 32, dtype=torch.float16)
    with pytest.raises(AssertionError):
        F.attention(q, k, k, False, 0.5, 64, 64)


def test_unsupported_head_dim_asserts_like_reference():
    q = torch.zeros(1, 1, 64, 48, dtype=torch.float16)
    with pytest.raises(AssertionError):
        F.attention(q, q, q, False, 0.5, 64, 64)


def test_cpu_tensors_are_rejected_not_computed():
    q = torch.zeros(1, 1, 64, 64, dtype=torch.float16)
    with pytest.raises(ValueError):
        F.attention(q, q, q, False, 0.5, 64, 64)


def test_unsupported_dtype_rejected():
    q = torch.zeros(1, 1, 64, 64, dtype=torch.float32)
    with pytest.raises(TypeError):
        F.forward(q, q, q, False, 0.5)


def test_get_tiling_returns_int_pair_for_any_valid_shape():
    for key in [(128, 8, 2048, 128, True), (32, 8, 2048, 128, False), (3, 5, 1000, 32, False),
                (1, 1, 1, 16, True), (4, 16, 8192, 64, True), (64, 8, 1024, 256, False)]:
        bm, bn = F.get_tiling(*key)
        assert isinstance(bm, int) and isinstance(bn, int)
        if key[-1]:
            assert bm % bn == 0


def test_get_tiling_errors():
    with pytest.raises(AssertionError):
        F.get_tiling(1, 1, 64, 48, False)
    with pytest.raises(ValueError):
        F.get_tiling(0, 1, 64, 64, False)


def test_resolve_tiling_rejects_reference_nan_tiling():
    # (64, 256) causal produced NaN in the reference (run_correctness_test.py:24-25)
    with pytest.raises(ValueError):
        F.resolve_tiling(256, True, 64, 256)
    assert F.resolve_tiling(256, False, 64, 256)[0] in (64, 128, 256)
