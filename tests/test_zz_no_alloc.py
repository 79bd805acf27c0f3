"""rsfa_attention_fwd_noalloc: the entry point that allocates nothing.

It runs the kernels of rsfa_attention_fwd with its queue counters and
workspace in the library's fixed per-device buffer, so its results must be
bitwise those of rsfa_attention_fwd on the same arguments.  Each case makes
two calls in a row on the same buffer, the second on a smaller problem, and
one case replays the call from a HIP graph.  The size check runs before any
device work and is tested without a GPU.
"""
import ctypes

import pytest
import torch

from ascend_rsfa import _native
from oracle import attention as A

_F8 = getattr(torch, "float8_e5m2", None)


def _args(q, k, v, o, lse, causal, scale, dtype_code, flags=0, ws=None):
    a = _native.FwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype = dtype_code
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    a.lse = lse.data_ptr() if lse is not None else 0
    a.z, a.h, a.n_ctx, a.head_dim = q.shape
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", o)):
        getattr(a, name)[:] = list(t.stride())
    a.sm_scale, a.causal, a.flags = scale, int(causal), flags
    if ws is not None:
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()
    return a


def _workspace_bytes(lib, a):
    """What rsfa_attention_fwd needs for `a`, with the tile its launch picks."""
    n = 0  # a float8 V needs none
    if a.causal and a.flags & _native.FLAG_CAUSAL_SPLIT:
        bm, bn = ctypes.c_int32(), ctypes.c_int32()
        assert lib.rsfa_get_tiling(a.z, a.h, a.n_ctx, a.head_dim, a.causal, a.dtype,
                                   ctypes.byref(bm), ctypes.byref(bn)) == 0
        n += int(lib.rsfa_split_workspace_bytes(a.z, a.h, a.n_ctx, a.head_dim, bm.value))
    return n


def _pair(shape, causal, scale, dtype, flags, seed):
    """Runs both entry points on one seeded input; returns (o, lse) of each."""
    lib = _native.lib()
    q, k, v = (t.cuda() for t in A.make_inputs(*shape, seed=seed))
    if dtype == "v8":
        v = v.to(_F8)
        code = _native.DTYPE_F16_V8E5M2
    elif dtype == torch.bfloat16:
        q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
        code = _native.DTYPE_BF16
    else:
        code = _native.DTYPE_F16
    res = []
    for entry in ("rsfa_attention_fwd", "rsfa_attention_fwd_noalloc"):
        o = torch.full_like(q, float("nan"))
        lse = torch.full(shape[:3], float("nan"), dtype=torch.float32, device="cuda")
        a = _args(q, k, v, o, lse, causal, scale, code, flags)
        ws = None
        if entry == "rsfa_attention_fwd":
            nbytes = _workspace_bytes(lib, a)
            if nbytes:
                ws = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
                a = _args(q, k, v, o, lse, causal, scale, code, flags, ws)
        else:
            a.workspace, a.workspace_bytes = 0, 0  # ignored by the no-allocation entry point
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        print(f"no-alloc: {entry} shape={shape} causal={causal} dtype={dtype} flags={flags:#x}", flush=True)
        st = getattr(lib, entry)(ctypes.byref(a), stream)
        assert st == 0, lib.rsfa_strerror(st).decode()
        torch.cuda.synchronize()
        res.append((o, lse, ws))
    return res


def _check_equal(res):
    (o0, l0, _), (o1, l1, _) = res
    assert not torch.isnan(o0.float()).any()
    assert torch.equal(o1, o0), f"max |diff| {(o1.float() - o0.float()).abs().max().item():.3e}"
    assert torch.equal(l1, l0)


CASES = [
    # (first shape, second smaller shape, causal, dtype, flags)
    ((2, 8, 1024, 128), (1, 4, 300, 128), False, torch.float16, 0),
    ((2, 8, 2048, 128), (1, 8, 640, 128), True, torch.float16, 0),
    ((1, 8, 1024, 128), (1, 2, 384, 128), True, torch.float16, _native.FLAG_CAUSAL_SPLIT),
    ((2, 4, 1024, 64), (1, 4, 200, 64), True, torch.bfloat16, 0),
    ((1, 8, 1024, 128), (1, 2, 256, 64), False, "v8", 0),
    ((1, 4, 1024, 128), (1, 2, 512, 128), True, "v8", _native.FLAG_CAUSAL_SPLIT),
    ((2, 8, 1024, 128), (1, 3, 500, 128), True, torch.float16, _native.FLAG_STATIC_SCHEDULE),
]


@pytest.mark.gpu
@pytest.mark.parametrize("big,small,causal,dtype,flags", CASES)
def test_noalloc_matches_the_allocating_entry_point_twice_in_a_row(big, small, causal, dtype, flags):
    if dtype == "v8" and _F8 is None:
        pytest.skip("torch has no float8_e5m2")
    for i, shape in enumerate((big, small)):
        _check_equal(_pair(shape, causal, 0.3 if i == 0 else -0.7, dtype, flags, seed=300 + i))


@pytest.mark.gpu
def test_noalloc_under_graph_capture():
    lib = _native.lib()
    shape = (2, 8, 1024, 128)
    q, k, v = (t.cuda() for t in A.make_inputs(*shape, seed=310))
    (o_ref, l_ref, _), _ = _pair(shape, True, 0.3, torch.float16, 0, seed=310)
    o = torch.empty_like(q)
    lse = torch.empty(shape[:3], dtype=torch.float32, device="cuda")
    a = _args(q, k, v, o, lse, True, 0.3, _native.DTYPE_F16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up before capture
        assert lib.rsfa_attention_fwd_noalloc(ctypes.byref(a), ctypes.c_void_p(side.cuda_stream)) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = lib.rsfa_attention_fwd_noalloc(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, lib.rsfa_strerror(st).decode()
    torch.cuda.synchronize()
    other = [t.cuda() for t in A.make_inputs(1, 2, 512, 64, seed=311)]
    for rep in range(4):
        print(f"no-alloc graph replay {rep}", flush=True)
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), f"replay {rep}"
        assert torch.equal(lse, l_ref), f"replay {rep}"
        # an eager no-alloc call on another problem between replays
        oo = torch.empty_like(other[0])
        b = _args(*other, oo, None, False, 0.5, _native.DTYPE_F16)
        assert lib.rsfa_attention_fwd_noalloc(ctypes.byref(b), ctypes.c_void_p(
            torch.cuda.current_stream().cuda_stream)) == 0
        torch.cuda.synchronize()
        assert not torch.isnan(oo.float()).any()


def _cpu_args(n=8192, d=128, **over):
    a = _native.FwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype = _native.DTYPE_F16
    a.q = a.k = a.v = a.o = 0x1000
    a.z, a.h, a.n_ctx, a.head_dim = 1, 8, n, d
    st = [8 * n * d, n * d, d, 1]
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, name)[:] = st
    a.sm_scale, a.causal = 0.5, 0
    for key, val in over.items():
        setattr(a, key, val)
    return a


def test_noalloc_rejects_problems_beyond_its_buffer_before_device_work():
    lib = _native.lib()
    limit = _native.NOALLOC_WORKSPACE_BYTES
    # split state: (2 + 64) fp32 per query row; 63488 rows (a multiple of
    # every BLOCK_M) fit the limit, 63744 do not
    fits = _cpu_args(z=1, h=1, n=63488, d=64, causal=1, flags=_native.FLAG_CAUSAL_SPLIT)
    assert lib.rsfa_split_workspace_bytes(1, 1, 63488, 64, 256) == 63488 * 66 * 4 <= limit
    over = _cpu_args(z=1, h=1, n=63744, d=64, causal=1, flags=_native.FLAG_CAUSAL_SPLIT)
    assert lib.rsfa_split_workspace_bytes(1, 1, 63744, 64, 256) > limit
    assert lib.rsfa_attention_fwd_noalloc(ctypes.byref(over), None) == _native.E_SCRATCH
    # a float8 V needs no workspace at any size or head dim
    big_v8 = _cpu_args(n=32768, d=32, dtype=_native.DTYPE_F16_V8E5M2, z=2)
    # split state: (2 + head_dim) fp32 per query row, rounded to the tile
    split = _cpu_args(z=8, h=32, n_ctx=16384, causal=1, flags=_native.FLAG_CAUSAL_SPLIT)
    assert lib.rsfa_attention_fwd_noalloc(ctypes.byref(split), None) == _native.E_SCRATCH
    assert "RSFA_NOALLOC_WORKSPACE_BYTES" in lib.rsfa_strerror(_native.E_SCRATCH).decode()
    # the same problems without workspace needs pass the size check
    assert lib.rsfa_attention_fwd_noalloc(None, None) == _native.E_NULL
    assert lib.rsfa_attention_fwd_noalloc(ctypes.byref(_cpu_args(struct_size=8)), None) == _native.E_ABI
    if not torch.cuda.is_available():
        for a in (fits, big_v8, _cpu_args(z=8, h=32, n_ctx=16384, causal=1), _cpu_args(z=64)):
            assert lib.rsfa_attention_fwd_noalloc(ctypes.byref(a), None) == _native.E_DEVICE
