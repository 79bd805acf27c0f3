"""CPU tests of the C ABI (librsfa.so): exports, host logic, argument checks.

Nothing here launches a kernel: every rsfa_attention_fwd call is rejected by
its argument checks before any device work, and the one call with valid
arguments only runs where no GPU is visible (it must fail with E_DEVICE).
"""
import ctypes
import os
import re

import pytest
import torch

from ascend_rsfa import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "rsfa.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rsfa_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    declared = _declared_functions()
    assert declared, "no functions parsed from include/rsfa.h"
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.SIGNATURES), "ctypes signature table out of sync with rsfa.h"


def test_abi_version_and_struct_layout():
    lib = _native.lib()
    assert lib.rsfa_abi_version() == _native.ABI_VERSION
    # struct rsfa_fwd_args: 4+4 + 6*8 ptr + 8 + 4*8 + 16*8 + 4*5
    assert ctypes.sizeof(_native.FwdArgs) == 8 + 48 + 8 + 32 + 128 + 24


def test_strerror_covers_all_codes():
    lib = _native.lib()
    codes = [0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11]
    msgs = [lib.rsfa_strerror(c).decode() for c in codes]
    assert len(set(msgs)) == len(codes)
    assert "unknown" in lib.rsfa_strerror(-99).decode()


def _tiling(z, h, n, d, causal, dtype=_native.DTYPE_F16):
    bm, bn = ctypes.c_int32(), ctypes.c_int32()
    st = _native.lib().rsfa_get_tiling(z, h, n, d, causal, dtype, ctypes.byref(bm), ctypes.byref(bn))
    return st, bm.value, bn.value


# the reference's get_tiling keys (flash_attention_forward.py:628-664) and the BASELINE configs
REFERENCE_KEYS = [
    (1, 1, 64, 64, False), (1, 1, 64, 64, True), (1, 1, 128, 128, False), (1, 1, 128, 128, True),
    (1, 2, 256, 256, False), (2, 2, 128, 256, False), (1, 2, 1024, 64, False), (1, 2, 1024, 64, True),
    (4, 32, 64, 64, False), (4, 32, 64, 64, True), (4, 32, 128, 128, False), (4, 32, 256, 128, True),
    (4, 32, 512, 64, True), (4, 32, 1024, 64, False), (4, 32, 1024, 64, True), (4, 32, 1024, 128, False),
    (4, 32, 2048, 64, True), (4, 32, 2048, 128, False), (4, 32, 4096, 64, False), (128, 8, 1024, 64, False),
    (128, 8, 1024, 128, True), (128, 8, 1024, 256, True), (128, 8, 2048, 128, True), (128, 8, 2048, 256, True),
    (128, 8, 4096, 128, True), (128, 8, 8192, 64, True), (128, 8, 1024, 128, False), (128, 8, 1024, 256, False),
    (128, 8, 2048, 128, False), (128, 8, 2048, 256, False), (128, 8, 4096, 128, False), (128, 8, 8192, 64, False),
    (2, 8, 1024, 128, True), (32, 8, 2048, 128, False), (64, 8, 1024, 256, False), (64, 8, 1024, 256, True),
    (4, 16, 8192, 64, True),
]


@pytest.mark.parametrize("key", REFERENCE_KEYS)
def test_get_tiling_answers_every_reference_and_baseline_shape(key):
    z, h, n, d, causal = key
    for dtype in (_native.DTYPE_F16, _native.DTYPE_BF16):
        st, bm, bn = _tiling(z, h, n, d, int(causal), dtype)
        assert st == 0
        assert bm in (64, 128, 256) and bn in (32, 64, 128)
        if causal:
            assert bm % bn == 0
        # deterministic, and a compiled instantiation resolve_tiling maps to itself
        assert _tiling(z, h, n, d, int(causal), dtype) == (0, bm, bn)
        rbm, rbn = ctypes.c_int32(), ctypes.c_int32()
        assert _native.lib().rsfa_resolve_tiling(d, int(causal), dtype, bm, bn, ctypes.byref(rbm),
                                                 ctypes.byref(rbn)) == 0
        assert (rbm.value, rbn.value) == (bm, bn)


def test_get_tiling_rejects_bad_shapes():
    assert _tiling(0, 1, 64, 64, 0)[0] == _native.E_SHAPE
    assert _tiling(1, 1, 0, 64, 0)[0] == _native.E_SHAPE
    assert _tiling(1, 1, 64, 48, 0)[0] == _native.E_HEADDIM
    assert _tiling(1, 1, 64, 64, 0, dtype=7)[0] == _native.E_DTYPE
    bm = ctypes.c_int32()
    assert _native.lib().rsfa_get_tiling(1, 1, 64, 64, 0, 0, ctypes.byref(bm), None) == _native.E_NULL


@pytest.mark.parametrize("req,causal,ok", [
    ((16, 16), False, True), ((64, 16), True, True), ((128, 512), False, True), ((64, 256), False, True),
    ((128, 64), True, True), ((16, 16), True, True),
    ((64, 256), True, False),    # causal BN > BM: NaN in the reference, rejected here
    ((48, 64), False, False),    # not a power of two
    ((8, 64), False, False),     # below 16
    ((512, 256), False, False),  # BM*BN > 65536
    ((1024, 16), False, False),  # above 512
])
def test_resolve_tiling_rules(req, causal, ok):
    bm, bn = ctypes.c_int32(), ctypes.c_int32()
    for d in (16, 32, 64, 128, 256):
        st = _native.lib().rsfa_resolve_tiling(d, int(causal), _native.DTYPE_F16, req[0], req[1],
                                               ctypes.byref(bm), ctypes.byref(bn))
        if ok:
            assert st == 0 and bm.value in (64, 128, 256) and bn.value in (32, 64, 128)
            if causal:
                assert bm.value % bn.value == 0
        else:
            assert st == _native.E_TILE


def test_split_workspace_bytes_matches_reference_state_shape():
    # reference: state = empty((2, Z, H, cdiv(N, BM), BM), fp32)  (flash_attention_forward.py:501),
    # then the un-normalised accumulator [Z, H, cdiv(N, BM), BM, D] in fp32, which the
    # reference rounds to the input dtype into O instead (353)
    lib = _native.lib()
    assert lib.rsfa_split_workspace_bytes(128, 8, 2048, 128, 128) == (2 + 128) * 128 * 8 * 16 * 128 * 4
    assert lib.rsfa_split_workspace_bytes(2, 3, 100, 64, 64) == (2 + 64) * 2 * 3 * 2 * 64 * 4
    assert lib.rsfa_split_workspace_bytes(0, 3, 100, 64, 64) == 0
    assert lib.rsfa_split_workspace_bytes(2, 3, 100, 48, 64) == 0


def test_v8_workspace_bytes_is_zero():
    """The kernels read a float8 V's bytes at every head dim: no copy."""
    lib = _native.lib()
    for d in (16, 32, 64, 128, 256, 48):
        assert lib.rsfa_v8_workspace_bytes(32, 8, 2048, d) == 0
    assert lib.rsfa_v8_workspace_bytes(0, 1, 17, 64) == 0


@pytest.mark.parametrize("causal", [0, 1])
def test_float8_v_dtype_has_the_fp16_tilings(causal):
    lib = _native.lib()
    for shape in [(32, 8, 2048, 128), (4, 16, 8192, 64), (64, 8, 1024, 256), (2, 8, 1024, 16)]:
        assert _tiling(*shape, causal, _native.DTYPE_F16_V8E5M2) == _tiling(*shape, causal)
    bm, bn = ctypes.c_int32(), ctypes.c_int32()
    assert lib.rsfa_resolve_tiling(128, causal, _native.DTYPE_F16_V8E5M2, 128, 64,
                                   ctypes.byref(bm), ctypes.byref(bn)) == 0


def _valid_args(**over):
    a = _native.FwdArgs()
    a.struct_size = ctypes.sizeof(_native.FwdArgs)
    a.dtype = _native.DTYPE_F16
    a.q = a.k = a.v = a.o = 0x1000
    a.z, a.h, a.n_ctx, a.head_dim = 2, 3, 128, 64
    st = [3 * 128 * 64, 128 * 64, 64, 1]
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = st
    a.sm_scale = 0.5
    a.causal = 0
    for k, v in over.items():
        if k.endswith("_stride"):
            getattr(a, k)[:] = v
        else:
            setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,code", [
    (dict(struct_size=8), _native.E_ABI),
    (dict(q=0), _native.E_NULL),
    (dict(o=0), _native.E_NULL),
    (dict(dtype=5), _native.E_DTYPE),
    (dict(head_dim=48), _native.E_HEADDIM),
    (dict(head_dim=512), _native.E_HEADDIM),
    (dict(z=0), _native.E_SHAPE),
    (dict(n_ctx=0), _native.E_SHAPE),
    (dict(k=0x1008), _native.E_ALIGN),
    (dict(v_stride=[3 * 128 * 64, 128 * 64, 64, 2]), _native.E_ALIGN),
    (dict(q_stride=[3 * 128 * 64, 128 * 64, 60, 1]), _native.E_ALIGN),
    (dict(lse=0x1002), _native.E_ALIGN),
    (dict(dtype=3), _native.E_DTYPE),
    # a float8 V needs 16-byte rows: outer strides a multiple of 16 elements
    (dict(dtype=_native.DTYPE_F16_V8E5M2, v_stride=[3 * 128 * 72, 128 * 72, 72, 1]), _native.E_ALIGN),
    # tile requests follow the reference's rules
    (dict(block_m=48, block_n=64), _native.E_TILE),
    (dict(block_m=64, block_n=256, causal=1), _native.E_TILE),
    # K/V row strides whose 128-row key tile (D=64) spans 4 GiB: the loader's
    # 32-bit per-lane offsets would wrap, so they are refused before launch
    (dict(k_stride=[0, 0, 16909320, 1]), _native.E_ALIGN),
    (dict(v_stride=[0, 0, 16909320, 1]), _native.E_ALIGN),
    # Q rows, loaded by the same loader into LDS by the ping-pong tiles
    (dict(q_stride=[0, 0, 16909320, 1]), _native.E_ALIGN),
    (dict(head_dim=256, k_stride=[0, 0, 69273664, 1]), _native.E_ALIGN),
    # the split state's rows are 32-bit: Z*H*N_CTX (rounded up to 256) < 2^31
    (dict(z=1024, h=1024, n_ctx=2048, causal=1, flags=_native.FLAG_CAUSAL_SPLIT), _native.E_SHAPE),
])
def test_attention_fwd_rejects_invalid_arguments(over, code):
    lib = _native.lib()
    assert lib.rsfa_attention_fwd(ctypes.byref(_valid_args(**over)), None) == code
    assert lib.rsfa_attention_fwd(None, None) == _native.E_NULL


def test_attention_fwd_without_gpu_reports_device_error():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible; this check needs a machine without one")
    lib = _native.lib()
    assert lib.rsfa_attention_fwd(ctypes.byref(_valid_args()), None) == _native.E_DEVICE


@pytest.mark.parametrize("over", [
    dict(k_stride=[0, 0, 16909312, 1]),            # the largest 8-multiple row stride whose 128-row tile fits
    dict(q_stride=[0, 0, 16909312, 1]),
    dict(head_dim=256, k_stride=[0, 0, 69273656, 1]),
    dict(z=1024, h=1024, n_ctx=2048, causal=1),     # fused causal has no split-state limit
    dict(block_m=128, block_n=64, causal=1),        # a valid request
])
def test_attention_fwd_limits_admit_the_boundary(over):
    """Arguments just inside the index limits pass every check made before
    device work: without a GPU the call gets as far as the device query."""
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible; this check needs a machine without one")
    lib = _native.lib()
    assert lib.rsfa_attention_fwd(ctypes.byref(_valid_args(**over)), None) == _native.E_DEVICE


def test_flag_constants_match_the_header():
    """The wrapper's flag bits are the header's RSFA_FLAG_* values."""
    hdr = open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "include", "rsfa.h")).read()
    flags = {m.group(1): int(m.group(2), 16) for m in re.finditer(r"#define RSFA_FLAG_(\w+)\s+(0x[0-9a-fA-F]+)u", hdr)}
    assert flags == {"STATIC_SCHEDULE": 1, "CAUSAL_SPLIT": 2, "EXACT_TILE": 4, "TILE_HINT": 8, "SINGLE_BLOCKS": 16}
    for name, val in flags.items():
        assert getattr(_native, "FLAG_" + name) == val
