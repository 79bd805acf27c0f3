"""Oracle functions (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

reference_attention / reference_lse
    Closed form, fp32 on the CPU, from the same fp16/bf16 inputs:
        O = softmax((Q K^T) * sm_scale + mask) V,   mask = -inf where key > query
    Follows the golden the reference tests against,
    benchmarks/run_correctness_test.py:68-92 (npu_fusion_attention, BNSD,
    sparse_mode=2 = left-up causal, i.e. query m sees keys 0..m), and the
    small kernels of ascend_rsfa/flash_attention_forward.py:84-88.
    The LSE is the reference's M = m + ln(l) (400-403): logsumexp of the
    scaled scores per query row.
    Pinned by (tests/test_oracle.py):
      * golden fixtures from a float64 brute-force loop (tests/golden/),
      * torch.nn.functional.scaled_dot_product_attention in float64,
      * closed forms: sm_scale = 0 gives the (prefix) mean of V; causal row 0
        returns V[0]; one-hot keys with a large scale retrieve one V row,
      * invariants: joint permutation of K/V rows (non-causal), rows of P are
        convex weights so min V <= O <= max V per column,
      * planted mistakes (shifted diagonal, dropped scale, transposed V,
        softmax over the wrong axis) each fail at least one of the above.

round_e5m2 / reference_attention_fp8v / fp8v_error_bound
    The reference's fp8_v branch (flash_attention_forward.py:208-211, 217,
    453-456, 466): with V in float8 e5m2, P = exp(S - m) is cast to e5m2 for
    P.V while the row sum l adds the unrounded P.  round_e5m2 restates the
    OCP e5m2 format (sign, 5 exponent bits with bias 15, 2 fraction bits,
    subnormals down to 2^-16, round to nearest even) from its definition.
    reference_attention_fp8v evaluates the branch with the exact row max (one
    key tile), fp8v_error_bound bounds any tiling of it: every P element is
    rounded with relative error <= 2^-3 (normal range) or absolute error
    <= 2^-17 (subnormal range, in units where the row max is >= 1).
    Pinned by (tests/test_oracle.py): torch's own float32 -> float8_e5m2
    conversion on values across every binade, ties and the subnormal range;
    every finite e5m2 value maps to itself; sm_scale = 0 gives the mean of V
    exactly; a two-key case (p = 1 and 0.6, 0.6 rounds to 0.625) tells the
    unrounded row sum (O = 0.625 / 1.6) from a rounded one (0.625 / 1.625).

reference_lse_rounded_p
    The row normalisation of this build's fp16/bf16 kernels: the row sum adds
    P rounded to the input dtype (the P that enters P.V), so each output row's
    weights sum to 1; the reference adds the unrounded P (217, 467).  The two
    differ by at most one rounding of P (2^-11 fp16, 2^-8 bf16 relative).
    Pinned by (tests/test_oracle.py): two keys with p = 1 and 0.6 give
    ln(1.60009765625) for fp16 and ln(1.6015625) for bf16 (0.6 rounded),
    against ln(1.6) for the reference's unrounded sum; and it stays within
    that rounding bound of reference_attention's LSE on random inputs.

blockwise_attention
    The reference's tiled algorithm with its rounding points (fp16 P, fp16
    round trip of the unnormalised prefix accumulator, -1e6 additive mask,
    FA4 rescale skip), restated in plain C in fa2_blockwise.c.
    Pinned against reference_attention within the repo tolerance and against
    the reference's published error statistics
    (benchmarks/correctness_test_results.txt:15-33: max |err| <= 9.77e-4 at
    N(0, 0.5^2) inputs, sm_scale 0.5).
"""
import ctypes
import math
import os

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libfa2_oracle.so")
_clib = None

# ~1 GiB of fp32 scores per chunk of heads
_CHUNK_BYTES = 1 << 30


def causal_mask(n, device="cpu"):
    """Boolean [n, n], True where key n' > query m (masked out)."""
    return torch.triu(torch.ones(n, n, dtype=torch.bool, device=device), diagonal=1)


def reference_attention(q, k, v, causal, sm_scale, return_lse=False, heads=None):
    """fp32 closed form on the CPU; q, k, v [Z, H, N, D] (any float dtype).

    ``heads``: optional list of (z, h) pairs; then only those heads are
    computed and the result is [len(heads), N, D] (and [len(heads), N] LSE).
    """
    Z, H, N, D = q.shape
    if heads is None:
        qf = q.reshape(Z * H, N, D)
        kf = k.reshape(Z * H, N, D)
        vf = v.reshape(Z * H, N, D)
    else:
        qf = torch.stack([q[z, h] for z, h in heads])
        kf = torch.stack([k[z, h] for z, h in heads])
        vf = torch.stack([v[z, h] for z, h in heads])
    qf = qf.detach().to("cpu", torch.float32)
    kf = kf.detach().to("cpu", torch.float32)
    vf = vf.detach().to("cpu", torch.float32)
    G = qf.shape[0]
    out = torch.empty((G, N, D), dtype=torch.float32)
    lse = torch.empty((G, N), dtype=torch.float32) if return_lse else None
    mask = causal_mask(N) if causal else None
    step = max(1, _CHUNK_BYTES // max(1, N * N * 4))
    for g0 in range(0, G, step):
        g1 = min(G, g0 + step)
        s = torch.matmul(qf[g0:g1], kf[g0:g1].transpose(-1, -2)) * float(sm_scale)
        if mask is not None:
            s.masked_fill_(mask, float("-inf"))
        if lse is not None:
            lse[g0:g1] = torch.logsumexp(s, dim=-1)
        p = torch.softmax(s, dim=-1)
        out[g0:g1] = torch.matmul(p, vf[g0:g1])
        del s, p
    if heads is None:
        out = out.reshape(Z, H, N, D)
        if lse is not None:
            lse = lse.reshape(Z, H, N)
    return (out, lse) if return_lse else out


E5M2_MAX = 57344.0  # 1.75 * 2^15, the largest finite e5m2


def round_e5m2(x):
    """Round to the nearest float8 e5m2 value (ties to even), returned as float32.

    e5m2: sign, 5 exponent bits (bias 15), 2 fraction bits.  Normal values
    1.f x 2^e for e in [-14, 15]; subnormals 0.f x 2^-14 (spacing 2^-16).
    Magnitudes that round above E5M2_MAX become inf.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, -14.0)  # below 2^-14 the spacing stays 2^-16
    q = np.exp2(e - 2.0)      # spacing of e5m2 values in the binade of a
    r = np.round(a / q) * q   # numpy rounds halves to even; a / q is exact
    r = np.where(r > E5M2_MAX, np.inf, r)
    r = np.where(np.isinf(a), np.inf, r)
    return (np.sign(x) * r).astype(np.float32)


def _heads_f32(q, k, v, heads):
    Z, H, N, D = q.shape
    if heads is None:
        heads = [(z, h) for z in range(Z) for h in range(H)]
    pick = lambda t: torch.stack([t[z, h] for z, h in heads]).detach().to("cpu", torch.float32)
    return pick(q), pick(k), pick(v), heads


def _scores_exp(qf, kf, causal, sm_scale):
    """p = exp(S - rowmax S) (masked keys 0), float64, with S in float32."""
    s = torch.matmul(qf, kf.transpose(-1, -2)) * float(sm_scale)
    if causal:
        s.masked_fill_(causal_mask(s.shape[-1]), float("-inf"))
    s = s.double()
    p = torch.exp(s - s.max(dim=-1, keepdim=True).values)
    return p


def reference_attention_fp8v(q, k, v8, causal, sm_scale, heads=None):
    """The reference's fp8_v branch with the exact row max (a single key
    tile): O = (e5m2(P) @ V) / sum(P), P = exp(S - max S); [len(heads), N, D]
    (all heads when ``heads`` is None, then reshaped to [Z, H, N, D])."""
    qf, kf, vf, hs = _heads_f32(q, k, v8.float(), heads)
    p = _scores_exp(qf, kf, causal, sm_scale)
    p8 = torch.from_numpy(round_e5m2(p.float().numpy())).double()
    out = (torch.matmul(p8, vf.double()) / p.sum(dim=-1, keepdim=True)).float()
    return out.reshape(q.shape) if heads is None else out


def fp8v_error_bound(q, k, v8, causal, sm_scale, heads=None):
    """Elementwise bound on |O - O_exact| for any tiling of the fp8_v branch,
    O_exact = softmax(S) V with V's e5m2 values: P rounding (2^-3 relative,
    2^-17 absolute in the subnormal range), fp32 accumulation, fp16 output."""
    qf, kf, vf, hs = _heads_f32(q, k, v8.float(), heads)
    p = _scores_exp(qf, kf, causal, sm_scale)
    av = vf.double().abs()
    l = p.sum(dim=-1, keepdim=True)
    vis = (p > 0).double() if causal else torch.ones_like(p)
    exact = torch.matmul(p, vf.double()) / l
    b = (0.126 * torch.matmul(p, av) + 2.0 ** -17 * torch.matmul(vis, av)) / l
    b = b + 2.0 ** -10 * exact.abs() + 1e-4
    b = b.float()
    return b.reshape(q.shape) if heads is None else b


def reference_lse_rounded_p(q, k, causal, sm_scale, heads=None):
    """Row logsumexp as this build's fp16/bf16 kernels normalise: the row sum
    adds P = exp(S - max S) rounded to the input dtype (the P that enters
    P.V), where the reference adds the unrounded P
    (flash_attention_forward.py:217, 467; ``reference_attention(...,
    return_lse=True)``).  Exact row max (every P <= 1); float64 result
    [len(heads), N] (all heads when ``heads`` is None, reshaped to [Z, H, N])."""
    qf, kf, _, hs = _heads_f32(q, k, k, heads)
    s = torch.matmul(qf, kf.transpose(-1, -2)) * float(sm_scale)
    if causal:
        s.masked_fill_(causal_mask(s.shape[-1]), float("-inf"))
    s = s.double()
    m = s.max(dim=-1, keepdim=True).values
    p = torch.exp(s - m).float().to(q.dtype).double()
    lse = (torch.log(p.sum(dim=-1, keepdim=True)) + m).squeeze(-1)
    return lse.reshape(q.shape[:3]) if heads is None else lse


def brute_force_attention_f64(q, k, v, causal, sm_scale):
    """Plain float64 loops over one head: q, k, v numpy [N, D].  Tiny inputs only."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    n, d = q.shape
    out = np.zeros((n, d))
    lse = np.zeros(n)
    for i in range(n):
        keys = range(i + 1) if causal else range(n)
        scores = [sum(q[i, t] * k[j, t] for t in range(d)) * sm_scale for j in keys]
        mx = max(scores)
        w = [math.exp(s - mx) for s in scores]
        tot = sum(w)
        lse[i] = mx + math.log(tot)
        for t in range(d):
            out[i, t] = sum(wj * v[j, t] for wj, j in zip(w, keys)) / tot
    return out, lse


def _load_clib():
    global _clib
    if _clib is None:
        if not os.path.exists(_LIB_PATH):
            from . import build_oracle

            build_oracle.build()
        lib = ctypes.CDLL(_LIB_PATH)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        lib.rsfa_oracle_fa2_forward.restype = ctypes.c_int
        lib.rsfa_oracle_fa2_forward.argtypes = [u16p, u16p, u16p, u16p, ctypes.POINTER(ctypes.c_float)] + [
            ctypes.c_int] * 4 + [ctypes.c_float] + [ctypes.c_int] * 4
        lib.rsfa_oracle_f32_to_f16.restype = ctypes.c_uint16
        lib.rsfa_oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.rsfa_oracle_f16_to_f32.restype = ctypes.c_float
        lib.rsfa_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.rsfa_oracle_f32_to_bf16.restype = ctypes.c_uint16
        lib.rsfa_oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        _clib = lib
    return _clib


def c_library():
    return _load_clib()


def blockwise_attention(q, k, v, causal, sm_scale, BM, BN, return_lse=False):
    """The reference's tiled forward (C restatement); q, k, v CPU fp16/bf16 [Z, H, N, D]."""
    lib = _load_clib()
    Z, H, N, D = q.shape
    bf16 = q.dtype == torch.bfloat16
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("blockwise_attention takes fp16 or bf16 inputs")

    def u16(t):
        return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)

    qa, ka, va = u16(q), u16(k), u16(v)
    oa = np.empty_like(qa)
    lse = np.empty((Z, H, N), dtype=np.float32) if (return_lse and not causal) else None
    p16 = ctypes.POINTER(ctypes.c_uint16)
    st = lib.rsfa_oracle_fa2_forward(
        qa.ctypes.data_as(p16), ka.ctypes.data_as(p16), va.ctypes.data_as(p16), oa.ctypes.data_as(p16),
        lse.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if lse is not None else None,
        Z, H, N, D, float(sm_scale), 1 if causal else 0, int(BM), int(BN), 1 if bf16 else 0)
    if st != 0:
        raise ValueError("shape not runnable by the reference's tiled algorithm "
                         "(N must divide by BM and BN; causal needs BN <= BM)")
    out = torch.from_numpy(oa.view(np.int16)).view(q.dtype).reshape(Z, H, N, D)
    if return_lse:
        return out, (torch.from_numpy(lse) if lse is not None else None)
    return out


def make_inputs(Z, H, N, D, seed, dtype=torch.float16, std=1.0):
    """Seeded Q, K, V ~ N(0, std^2) drawn in fp32 on the CPU, then cast (q, k, v order)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    shape = (Z, H, N, D)
    q = (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype)
    k = (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype)
    v = (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype)
    return q, k, v


def fingerprint(*tensors):
    """SHA-256 of the raw bytes of the tensors (to check inputs match across machines)."""
    import hashlib

    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().to("cpu").contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()
