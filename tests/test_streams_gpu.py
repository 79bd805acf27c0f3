"""Launches the dynamic task queue cannot serve: graph capture and the
per-thread default stream.

The dynamic queue's ticket counter is found by stream handle and relies on one
stream running its launches in order.  A launch recorded into a HIP graph may
later be replayed on any stream, concurrently with replays of other graphs
captured on the same stream, and hipStreamPerThread is one handle for every
thread's stream; those launches run the static schedule, which gives bitwise
the results of the dynamic one.  Each replay is checked against the eager
result, with eager work and synchronisations between replays.
"""
import ctypes

import pytest
import torch

from ascend_rsfa import _native
from ascend_rsfa import flash_attention_forward as F
from oracle import attention as A

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("causal", [False, True])
def test_graphs_replayed_concurrently_on_two_streams(causal):
    inputs = [[t.cuda() for t in A.make_inputs(2, 8, 1024, 128, seed=s)] for s in (91, 92)]
    eager = [F.forward(q, k, v, causal, 0.3) for q, k, v in inputs]
    torch.cuda.synchronize()
    # warm up on a side stream before capture, as torch's graph docs ask
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for q, k, v in inputs:
            F.forward(q, k, v, causal, 0.3)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    # both graphs captured on torch's default capture stream
    graphs, outs = [], []
    for q, k, v in inputs:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(F.forward(q, k, v, causal, 0.3))
        graphs.append(g)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(4):
        print(f"graph replay {rep} causal={causal}", flush=True)
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        for g, s in zip(graphs, streams):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}: max |diff| {(o.float() - e.float()).abs().max().item():.3e}"
        # eager launches on the dynamic queue between replays
        again = F.forward(*inputs[rep % 2], causal, 0.3)
        torch.cuda.synchronize()
        assert torch.equal(again, eager[rep % 2])


def test_per_thread_default_stream():
    q, k, v = (t.cuda() for t in A.make_inputs(2, 8, 1024, 128, seed=93))
    eager = F.forward(q, k, v, True, 0.3)
    o = torch.full_like(q, float("nan"))
    a = _native.FwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype = _native.DTYPE_F16
    a.q, a.k, a.v, a.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    a.z, a.h, a.n_ctx, a.head_dim = q.shape
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", o)):
        getattr(a, name)[:] = list(t.stride())
    a.sm_scale = 0.3
    a.causal = 1
    torch.cuda.synchronize()
    per_thread = ctypes.c_void_p(2)  # hipStreamPerThread
    for _ in range(3):
        assert _native.lib().rsfa_attention_fwd(ctypes.byref(a), per_thread) == 0
    torch.cuda.synchronize()  # a device-wide synchronisation waits for the per-thread stream too
    assert torch.equal(o, eager)
