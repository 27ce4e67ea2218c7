"""The public operators captured in HIP graphs (torch.cuda.graph).

The kernels neither allocate nor synchronize, and with host cu_seqlens
(varlen) or the prepared index tables with validate=False (absorb) the
Python layer makes no host round trip once a call has cached its plan: one
eager call, then the same call captured and replayed.  Between replays the
inputs are overwritten in place (eager work on the same stream), and every
replay is checked bit for bit against an eager call on the new inputs.
"""
import math

import pytest
import torch

from varlenabsorbflashattn_amd import (packed_varlen_attn, prepare_target_attn_indices,
                                       target_attn_inner)
from varlenabsorbflashattn_amd.workloads import cu_from_lens

pytestmark = pytest.mark.gpu


def _replays(graph, out, refill, eager, n=3):
    for i in range(n):
        refill(i)
        want = eager()
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"  replay {i}", flush=True)
        assert torch.equal(out, want)


def test_varlen_forward_under_graph_capture(device):
    """Forward with split-K partials and combine (long key ranges) and plain
    items, 256-row tiles, host cu_seqlens."""
    q_lens, k_lens, H, D = [300, 16, 9], [700, 9000, 30000], 8, 128
    g = torch.Generator(device=device).manual_seed(3)
    Tq, Tk = sum(q_lens), sum(k_lens)
    q, k, v = (torch.randn(T, H, D, generator=g, device=device).to(torch.bfloat16)
               for T in (Tq, Tk, Tk))
    cq, ck = cu_from_lens(q_lens), cu_from_lens(k_lens)  # host tensors
    scale = 1.0 / math.sqrt(D)

    def call():
        with torch.no_grad():
            return packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck, scale=scale)

    print(f"[varlen graph] q={q_lens} k={k_lens} H={H} D={D}", flush=True)
    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()

    def refill(i):
        q.copy_(torch.randn(q.shape, generator=g, device=device).to(torch.bfloat16))
        v.mul_(-1.0)

    _replays(graph, out, refill, lambda: call().clone())


def test_absorb_forward_under_graph_capture(device):
    """Inner absorb forward on the prepared-index contract (validate=False):
    multi-workgroup samples and a W_V re-layout launch inside the graph."""
    q_lens, k_lens, H, D_H, F = [5, 20, 1, 9], [300, 2000, 64, 900], 8, 32, 256
    g = torch.Generator(device=device).manual_seed(4)
    Tq, Tk = sum(q_lens), sum(k_lens)
    u = (torch.randn(Tq, H, F, generator=g, device=device) * 0.1).to(torch.bfloat16)
    X = torch.randn(Tk, F, generator=g, device=device).to(torch.bfloat16)
    W_V = (torch.randn(F, H, D_H, generator=g, device=device) * 0.1).to(torch.bfloat16)
    cq, ck = cu_from_lens(q_lens).to(device), cu_from_lens(k_lens).to(device)
    qi, ki = prepare_target_attn_indices(cq, ck)
    scale = 1.0 / math.sqrt(D_H)

    def call():
        with torch.no_grad():
            return target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)

    print(f"[absorb graph] q={q_lens} k={k_lens} H={H} D_H={D_H} F={F}", flush=True)
    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()

    def refill(i):
        X.copy_(torch.randn(X.shape, generator=g, device=device).to(torch.bfloat16))
        W_V.mul_(0.5)

    _replays(graph, out, refill, lambda: call().clone())


def test_varlen_training_step_under_graph_capture(device):
    """Forward and backward (autograd) captured together, as a training step
    would be: warm-up iterations on a side stream, then capture; after each
    replay on new inputs the static gradients equal an eager step's."""
    q_lens, k_lens, H, D = [200, 7, 64], [180, 5000, 64], 4, 64
    g = torch.Generator(device=device).manual_seed(6)
    Tq, Tk = sum(q_lens), sum(k_lens)

    def rnd(T):
        return torch.randn(T, H, D, generator=g, device=device).to(torch.bfloat16)

    q, k, v = (rnd(T).requires_grad_(True) for T in (Tq, Tk, Tk))
    do = rnd(Tq)
    cq, ck = cu_from_lens(q_lens), cu_from_lens(k_lens)

    def step(q_, k_, v_):
        o = packed_varlen_attn(q_, k_, v_, cu_seqlens_q=cq, cu_seqlens_k=ck)
        o.backward(do)
        return o

    print(f"[varlen graph fwd+bwd] q={q_lens} k={k_lens} H={H} D={D}", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            q.grad = k.grad = v.grad = None
            step(q, k, v)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    q.grad = k.grad = v.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_static = step(q, k, v)

    for i in range(3):
        with torch.no_grad():
            q.copy_(rnd(Tq))
            k.mul_(-1.0)
        qe, ke, ve = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o_e = step(qe, ke, ve)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"  replay {i}", flush=True)
        assert torch.equal(o_static, o_e)
        for a, b in ((q.grad, qe.grad), (k.grad, ke.grad), (v.grad, ve.grad)):
            assert torch.equal(a, b)
