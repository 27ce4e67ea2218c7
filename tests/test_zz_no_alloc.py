"""vafa_varlen_fwd_noalloc: the varlen forward with its split-partial
workspace in a static device array instead of caller memory.

Checked through the C ABI against vafa_varlen_fwd with a workspace (bit for
bit: same kernels) and against the oracle (tests/parity.py bound), on two
calls in a row of which the second needs less scratch; plus the size limit,
which the entry point enforces on the host before any device call.
"""
import ctypes as C
import math

import numpy as np
import pytest
import torch

from oracle import varlen as ov
from parity import assert_close
from varlenabsorbflashattn_amd import _lib

# (q_lens, k_lens, H, D): the first call uses more scratch than the second
CALLS = [
    ([16, 1, 9, 12], [32768, 30000, 4000, 1024], 8, 128),
    ([150, 20], [9000, 5000], 4, 64),
]


def _cu(lens):
    c = np.zeros(len(lens) + 1, dtype=np.int64)
    c[1:] = np.cumsum(lens)
    return c


def _fwd_both(q_lens, k_lens, H, D, device):
    g = torch.Generator(device=device).manual_seed(sum(q_lens))
    Tq, Tk = sum(q_lens), sum(k_lens)
    q, k, v = (torch.randn(T, H, D, generator=g, device=device).to(torch.bfloat16)
               for T in (Tq, Tk, Tk))
    cq, ck = _cu(q_lens), _cu(k_lens)
    plan = _lib.device_plan("varlen", cq, ck, (H, D), device)
    L = _lib.lib()
    need = L.vafa_varlen_fwd_workspace(plan.info, D)
    print(f"[noalloc] q={q_lens} k={k_lens} H={H} D={D} scratch={need} B", flush=True)
    assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    o1, o2 = torch.empty_like(q), torch.full_like(q, float("nan"))
    lse1 = torch.empty(Tq, H, dtype=torch.float32, device=device)
    lse2 = torch.full_like(lse1, float("nan"))
    scale = 1.0 / math.sqrt(D)
    st = _lib.stream_ptr(device)
    _lib.check(L.vafa_varlen_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o1.data_ptr(),
                                 lse1.data_ptr(), plan.items.data_ptr(), plan.info, D,
                                 _lib.DT_BF16, scale, ws.data_ptr(), need, st))
    _lib.check(L.vafa_varlen_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o2.data_ptr(),
                                         lse2.data_ptr(), plan.items.data_ptr(), plan.info, D,
                                         _lib.DT_BF16, scale, st))
    torch.cuda.synchronize()
    return (q, k, v, cq, ck, scale), (o1, lse1), (o2, lse2)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_on_two_calls(device):
    for q_lens, k_lens, H, D in CALLS:
        (q, k, v, cq, ck, scale), (o1, lse1), (o2, lse2) = _fwd_both(q_lens, k_lens, H, D,
                                                                     device)
        assert torch.equal(o1, o2) and torch.equal(lse1, lse2)
        o_r, lse_r = ov.forward(*(t.float().cpu().numpy() for t in (q, k, v)), cq, ck, scale,
                                np.float64)
        assert_close("o", o2, o_r)
        assert_close("lse", lse2, lse_r, dtype=torch.bfloat16)


@pytest.mark.gpu
def test_noalloc_d16_matches_oracle(device):
    """16-bit D=16: vafa_varlen_fwd runs it on the D=32 matrix-core kernels over
    zero-padded copies, this entry point on the wave-per-row kernels (no room
    for the copies in the scratch): each is checked against the oracle with
    the parity bound, and the two against each other with the same bound."""
    (q, k, v, cq, ck, scale), (o1, lse1), (o2, lse2) = _fwd_both(
        [16, 3, 40], [5000, 900, 130], 4, 16, device)
    o_r, lse_r = ov.forward(*(t.float().cpu().numpy() for t in (q, k, v)), cq, ck, scale,
                            np.float64)
    for name, o in (("o ws", o1), ("o noalloc", o2)):
        assert_close(name, o, o_r)
    assert_close("lse", lse2, lse_r, dtype=torch.bfloat16)
    assert_close("o vs o", o2, o1.float().cpu().numpy())


@pytest.mark.gpu
def test_noalloc_under_graph_capture(device):
    """One eager call (which looks the scratch address up), then the same call
    captured with torch.cuda.graph and replayed three times, with eager work on
    the outputs between the replays: every replay equals the eager result bit
    for bit."""
    q_lens, k_lens, H, D = [16, 1, 9, 12], [32768, 30000, 4000, 1024], 8, 128
    g = torch.Generator(device=device).manual_seed(5)
    Tq, Tk = sum(q_lens), sum(k_lens)
    q, k, v = (torch.randn(T, H, D, generator=g, device=device).to(torch.bfloat16)
               for T in (Tq, Tk, Tk))
    plan = _lib.device_plan("varlen", _cu(q_lens), _cu(k_lens), (H, D), device)
    L = _lib.lib()
    o = torch.empty_like(q)
    lse = torch.empty(Tq, H, dtype=torch.float32, device=device)
    scale = 1.0 / math.sqrt(D)

    def call():
        return L.vafa_varlen_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                         lse.data_ptr(), plan.items.data_ptr(), plan.info, D,
                                         _lib.DT_BF16, scale, _lib.stream_ptr(device))

    print(f"[noalloc graph] q={q_lens} k={k_lens} H={H} D={D}", flush=True)
    _lib.check(call())
    torch.cuda.synchronize()
    o_eager, lse_eager = o.clone(), lse.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = call()
    _lib.check(rc)
    for i in range(3):
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"  replay {i}", flush=True)
        assert torch.equal(o, o_eager) and torch.equal(lse, lse_eager)


def test_noalloc_rejects_plans_beyond_the_scratch():
    """A plan whose split partials exceed the static scratch is refused on the
    host, before any device call (so this runs without a GPU)."""
    q_lens, k_lens, H, D = [16] * 600, [32768] * 600, 32, 128
    plan = _lib.plan_varlen(_cu(q_lens), _cu(k_lens), H, D)
    L = _lib.lib()
    need = L.vafa_varlen_fwd_workspace(C.byref(plan.info), D)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    rc = L.vafa_varlen_fwd_noalloc(None, None, None, None, None, None, C.byref(plan.info), D,
                                   _lib.DT_BF16, 1.0, None)
    assert rc == _lib.VAFA_ERR_WORKSPACE
    assert "static scratch holds 67108864" in _lib.last_error()
