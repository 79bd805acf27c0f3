"""FlashAttention-2 forward on MI355X (gfx950) behind the reference's Python surface.

Drop-in for ``ascend_rsfa/flash_attention_forward.py`` of Dell710000/ascend-rsfa:

==============================  ===============================================
this module                     reference (flash_attention_forward.py)
==============================  ===============================================
``get_num_compute_cores()``     ``get_num_compute_cores`` (19-21)
``_attention``                  ``class _attention(torch.autograd.Function)``
                                (547-616): same forward signature
                                ``(ctx, q, k, v, causal, sm_scale, BM, BN)``,
                                same assertions (553-554), same saved tensors
                                (612-615), no backward (calling it raises)
``attention``                   ``attention = _attention.apply`` (622)
``get_tiling(Z,H,N,D,causal)``  ``get_tiling`` (624-665): a lookup table there,
                                a gfx950 tile search here; returns
                                ``(BLOCK_M, BLOCK_N)`` for every valid shape
==============================  ===============================================

All arithmetic runs in the HIP library ``lib/librsfa.so`` (C ABI in
``include/rsfa.h``), enqueued on the current HIP stream of the tensors'
device.  There is no fallback path: without the built library, or for tensors
that are not on a GPU, the calls raise.

A ``float8_e5m2`` V with float16 Q and K runs the reference's fp8_v branch
(_attn_fwd_inner 208-211, 217): P is rounded to e5m2 for P.V while the row
sums add the unrounded P; O is float16.  The library widens V to fp16 in a
workspace first (exact: an e5m2 byte is the high byte of that fp16).

Behaviour beyond the reference (documented, deliberate):

* ``BM``/``BN`` keep the reference's meaning (query rows per program, keys per
  inner tile) and its validity rules; gfx950 runs them on the nearest compiled
  tile shape (``resolve_tiling``).  Causal calls with ``BN > BM``, which give
  NaN in the reference (benchmarks/run_correctness_test.py:24-25), raise
  ``ValueError`` instead.
* Any ``N_CTX >= 1`` works (the reference has no load masks, so it needs
  ``N_CTX`` divisible by its tiles).
* Per-tensor strides are honoured as long as the head dim is unit-stride; other
  layouts are copied to contiguous first.
"""
import ctypes

import torch

from . import _native

__all__ = ["attention", "get_tiling", "get_num_compute_cores", "resolve_tiling", "forward",
           "split_workspace_bytes"]

_DTYPES = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16}
_FP8_E5M2 = getattr(torch, "float8_e5m2", None)


def _raise_for(status):
    """Map an rsfa_status to the exception type the reference would raise."""
    if status == _native.OK:
        return
    msg = _native.strerror(status)
    if status == _native.E_HEADDIM:
        raise AssertionError(msg)
    if status == _native.E_DTYPE:
        raise TypeError(msg)
    if status in (_native.E_TILE, _native.E_SHAPE, _native.E_WORKSPACE, _native.E_ALIGN, _native.E_NULL):
        raise ValueError(msg)
    raise RuntimeError(f"rsfa error {status}: {msg}")


def get_num_compute_cores():
    """Compute units of the current device (reference 19-21 reads num_aicore)."""
    n = _native.lib().rsfa_get_num_compute_cores(torch.cuda.current_device())
    if n < 0:
        _raise_for(n)
    return n


def get_tiling(Z, H, N_CTX, HEAD_DIM, causal):
    """Return (BLOCK_M, BLOCK_N) for the shape (reference 624-665).

    The reference looks the shape up in a table of Ascend tilings and raises
    KeyError for any shape not listed.  Here a measured, correctness-gated
    tiling cache answers first when one is active (``tiling.use_cache`` or
    ``RSFA_TILING_CACHE``; entries that are not a compiled tile shape are
    ignored); otherwise the library searches the compiled gfx950 tile shapes
    with a register/LDS feasibility check and a makespan model of the
    persistent grid, so it answers for every valid shape.
    """
    from . import tiling
    cache = tiling.active_cache()
    if cache is not None:
        hit = cache.lookup(Z, H, N_CTX, HEAD_DIM, causal)
        if hit is not None:
            try:
                if resolve_tiling(HEAD_DIM, causal, hit[0], hit[1]) == tuple(hit):
                    return tuple(hit)
            except ValueError:
                pass
    bm = ctypes.c_int32()
    bn = ctypes.c_int32()
    st = _native.lib().rsfa_get_tiling(int(Z), int(H), int(N_CTX), int(HEAD_DIM), 1 if causal else 0,
                                       _native.DTYPE_F16, ctypes.byref(bm), ctypes.byref(bn))
    _raise_for(st)
    return (bm.value, bn.value)


def resolve_tiling(HEAD_DIM, causal, BM, BN, dtype=torch.float16):
    """The (BLOCK_M, BLOCK_N) instantiation that runs a request of (BM, BN)."""
    bm = ctypes.c_int32()
    bn = ctypes.c_int32()
    st = _native.lib().rsfa_resolve_tiling(int(HEAD_DIM), 1 if causal else 0, _DTYPES.get(dtype, -1),
                                           int(BM), int(BN), ctypes.byref(bm), ctypes.byref(bn))
    _raise_for(st)
    return (bm.value, bn.value)


def split_workspace_bytes(Z, H, N_CTX, HEAD_DIM, BM):
    return int(_native.lib().rsfa_split_workspace_bytes(int(Z), int(H), int(N_CTX), int(HEAD_DIM), int(BM)))


def _meets_contract(t):
    # 16-byte rows: outer strides a multiple of 8 two-byte or 16 one-byte elements
    mult = 16 // t.element_size()
    st = t.stride()
    return st[3] == 1 and all(s % mult == 0 for s in st[:3]) and t.data_ptr() % 16 == 0


def _as_kernel_layout(t):
    if _meets_contract(t):
        return t
    t = t.contiguous()
    if not _meets_contract(t):
        t = t.clone(memory_format=torch.contiguous_format)
    return t


def forward(q, k, v, causal, sm_scale, BM=0, BN=0, *, return_lse=False, split=False,
            static_schedule=False, out=None):
    """Run the forward kernel; returns ``o`` or ``(o, lse)``.

    ``BM = BN = 0`` lets the library pick the tiling.  ``split=True`` (causal
    only) runs the reference's two-launch prefix/diagonal split with an fp32
    state workspace; ``static_schedule=True`` replaces the dynamic task queue
    by the reference's grid-stride order (results are bitwise identical).
    ``lse`` is the natural-log logsumexp of the scaled scores, fp32 [Z, H, N].
    """
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share one 4-D shape [Z, H, N_CTX, D]; got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    # a float8 e5m2 V with float16 Q, K takes the reference's fp8_v branch (208-211)
    v8 = v.dtype == _FP8_E5M2 and q.dtype == torch.float16 and k.dtype == torch.float16
    if not v8 and not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k and v must have the same dtype (or float16 q, k with a float8_e5m2 v)")
    if q.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {q.dtype}; float16 and bfloat16 are supported")
    if not (q.is_cuda and k.is_cuda and v.is_cuda) or not (q.device == k.device == v.device):
        raise ValueError("q, k and v must be GPU tensors on one device")
    Z, H, N, D = q.shape
    lib = _native.lib()
    q_, k_, v_ = _as_kernel_layout(q), _as_kernel_layout(k), _as_kernel_layout(v)
    if out is None:
        o = torch.empty_like(q_)
    else:
        o = out
        if o.shape != q.shape or o.dtype != q.dtype or o.device != q.device or not _meets_contract(o):
            raise ValueError("out must match q's shape, dtype and device and have a unit-stride head dim")
    lse = torch.empty((Z, H, N), dtype=torch.float32, device=q.device) if return_lse else None

    args = _native.FwdArgs()
    args.struct_size = ctypes.sizeof(_native.FwdArgs)
    args.dtype = _native.DTYPE_F16_V8E5M2 if v8 else _DTYPES[q.dtype]
    args.q, args.k, args.v, args.o = q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr()
    args.lse = lse.data_ptr() if lse is not None else None
    args.z, args.h, args.n_ctx, args.head_dim = Z, H, N, D
    for name, t in (("q_stride", q_), ("k_stride", k_), ("v_stride", v_), ("o_stride", o)):
        getattr(args, name)[:] = list(t.stride())
    args.sm_scale = float(sm_scale)
    args.causal = 1 if causal else 0
    args.block_m = int(BM)
    args.block_n = int(BN)
    args.flags = (_native.FLAG_STATIC_SCHEDULE if static_schedule else 0) | (
        _native.FLAG_CAUSAL_SPLIT if (split and causal) else 0)
    ws = None
    with torch.cuda.device(q.device):
        # workspace: the fp16 copy of a float8 V, then the split state
        nbytes = int(lib.rsfa_v8_workspace_bytes(Z, H, N, D)) if v8 else 0
        if split and causal:
            bm = BM
            if not (BM or BN):
                bm, _ = get_tiling(Z, H, N, D, causal)
            else:
                bm, _ = resolve_tiling(D, causal, BM, BN, q.dtype)
            nbytes += split_workspace_bytes(Z, H, N, D, bm)
        if nbytes:
            ws = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
            args.workspace = ws.data_ptr()
            args.workspace_bytes = nbytes
        stream = torch.cuda.current_stream(q.device).cuda_stream
        st = lib.rsfa_attention_fwd(ctypes.byref(args), ctypes.c_void_p(stream))
    _raise_for(st)
    if out is not None and o is not out:
        out.copy_(o)
        o = out
    return (o, lse) if return_lse else o


# ============================================================================
# Same class name and apply alias as the reference (545-546, 619-622).
# ============================================================================
class _attention(torch.autograd.Function):

    @staticmethod
    def forward(ctx, q, k, v, causal, sm_scale, BM, BN):
        HEAD_DIM_Q, HEAD_DIM_K = q.shape[-1], k.shape[-1]
        HEAD_DIM_V = v.shape[-1]
        assert HEAD_DIM_Q == HEAD_DIM_K and HEAD_DIM_K == HEAD_DIM_V
        assert HEAD_DIM_K in {16, 32, 64, 128, 256}

        Z, H, N_CTX, HEAD_DIM = q.shape
        if causal:
            # the reference keeps a (1,) placeholder for the causal path (559-560)
            o = forward(q, k, v, True, sm_scale, BM, BN)
            M = torch.empty((1,), dtype=torch.float32, device=q.device)
        else:
            # non-causal writes the row logsumexp M = m + ln(l) (400-403)
            o, M = forward(q, k, v, False, sm_scale, BM, BN, return_lse=True)

        ctx.save_for_backward(q, k, v, o, M)
        ctx.sm_scale = sm_scale
        ctx.HEAD_DIM = HEAD_DIM_K
        ctx.causal = causal
        return o


attention = _attention.apply
