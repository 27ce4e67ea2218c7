"""GPU parity on the benchmark workloads themselves.

Every configuration that bench.py times is checked here on its own shape and
plan, against the numpy oracle in float32 on the host (the north-star
reference precision) with the tolerances of tests/parity.py:
  * configs[1] (C2): the whole 64-sequence H=16 D=128 batch, O and all grads;
  * configs[2] (C3): a seeded 24-sequence subset at H=32 D=128 that holds the
    longest key range and both extreme query lengths, plus the 4-16 key chunks
    per (sequence, head) that the config prescribes;
  * configs[3] (C4): all 2048 samples, inner forward and backward;
  * configs[4] (C5): the full 8192-sample forward (its own plan), with the
    output rows of 256 samples -- every sample at the 8192-key cap with the
    most queries among them -- compared against the oracle.
Inputs follow varlenabsorbflashattn_amd.workloads (the generator bench.py uses).
"""
import math

import numpy as np
import pytest
import torch

from oracle import absorb as oa
from oracle import varlen as ov
from parity import assert_close
from varlenabsorbflashattn_amd import (_lib, packed_varlen_attn, prepare_target_attn_indices,
                                       target_attn_inner)
from varlenabsorbflashattn_amd import workloads as W
from varlenabsorbflashattn_amd.absorb import _project_u

pytestmark = pytest.mark.gpu


def _host(t):
    return t.detach().float().cpu().numpy()


def _cu_np(lens):
    c = np.zeros(len(lens) + 1, dtype=np.int64)
    c[1:] = np.cumsum(lens)
    return c


def test_c2_full_size_fwd_bwd(device):
    case = W.config2(seed=0)
    print(f"[C2 full] H={case.H} D={case.D} n={len(case.q_lens)} sum_L={sum(case.q_lens)} "
          f"max_L={max(case.q_lens)}", flush=True)
    q, k, v, do = W.varlen_tensors(case, device, with_grad_out=True)
    cu = W.cu_from_lens(case.q_lens, device)
    qd, kd, vd = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = packed_varlen_attn(qd, kd, vd, cu_seqlens_q=cu, cu_seqlens_k=cu)
    o.backward(do)
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(case.D)
    hq, hk, hv, hdo = (_host(t) for t in (q, k, v, do))
    cu_h = _cu_np(case.q_lens)
    o_r, _ = ov.forward(hq, hk, hv, cu_h, cu_h, scale, np.float32)
    dq_r, dk_r, dv_r = ov.backward(hq, hk, hv, hdo, cu_h, cu_h, scale, np.float32)
    for n, a, r in (("o", o, o_r), ("dq", qd.grad, dq_r), ("dk", kd.grad, dk_r),
                    ("dv", vd.grad, dv_r)):
        assert_close(n, a, r)


def _c3_subset(n_keep=24):
    """Indices of a C3 subset: the longest key range, a 1-query and a
    16-query sequence, then the first sequences of the draw."""
    full = W.config3(seed=0)
    lq, lk = np.asarray(full.q_lens), np.asarray(full.k_lens)
    pick = [int(np.argmax(lk)), int(np.flatnonzero(lq == 1)[0]), int(np.flatnonzero(lq == 16)[0])]
    for i in range(len(lq)):
        if len(pick) >= n_keep:
            break
        if i not in pick:
            pick.append(i)
    pick.sort()
    return full, pick


def test_c3_subset_split_forward(device):
    full, pick = _c3_subset()
    q_lens = [full.q_lens[i] for i in pick]
    k_lens = [full.k_lens[i] for i in pick]
    case = W.VarlenCase("c3_subset", q_lens, k_lens, full.H, full.D, torch.bfloat16, seed=3)
    print(f"[C3 subset] H={case.H} D={case.D} n={len(pick)} max_Lk={max(k_lens)} "
          f"Lq in [{min(q_lens)},{max(q_lens)}]", flush=True)
    assert max(k_lens) >= 30000 and 1 in q_lens and 16 in q_lens
    # the config's 4-16 key chunks per (sequence, head)
    plan = _lib.plan_varlen(_cu_np(q_lens), _cu_np(k_lens), case.H, case.D)
    fwd = plan.section("fwd")
    assert len(fwd) and np.all(fwd[:, 4] >= 0), "every C3 tile runs split"
    assert fwd[:, 7].min() >= 4 and fwd[:, 7].max() <= 16
    assert plan.info.n_comb == len(pick)
    q, k, v = W.varlen_tensors(case, device)
    cq, ck = W.cu_from_lens(q_lens, device), W.cu_from_lens(k_lens, device)
    with torch.no_grad():
        o = packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)
    torch.cuda.synchronize()
    o_r, _ = ov.forward(_host(q), _host(k), _host(v), _cu_np(q_lens), _cu_np(k_lens),
                        1.0 / math.sqrt(case.D), np.float32)
    assert_close("o", o, o_r)


def _absorb_inputs(case, device, dtype=None):
    q_raw, X, W_Q, W_K, W_V = W.absorb_tensors(case, device, dtype=dtype)
    with torch.no_grad():
        u = _project_u(q_raw, W_Q, W_K).contiguous()
    del q_raw
    return u, X, W_V


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_c4_full_fwd_bwd(device, dtype):
    """bf16 (the benchmark) and fp32, the reference's documented call (no bf16
    flag: fp32 inputs, IEEE fp32 products)."""
    case = W.config4(seed=0)
    print(f"[C4 full {dtype}] samples={len(case.q_lens)} T_q={sum(case.q_lens)} "
          f"T_k={sum(case.k_lens)}", flush=True)
    u, X, W_V = _absorb_inputs(case, device, dtype)
    cq, ck = W.cu_from_lens(case.q_lens, device), W.cu_from_lens(case.k_lens, device)
    qi, ki = prepare_target_attn_indices(cq, ck)
    g = torch.Generator(device=device).manual_seed(11)
    dO = torch.randn(u.shape[0], case.H, case.D_H, generator=g, device=device).to(u.dtype)
    ud, Xd, Wd = (t.detach().clone().requires_grad_(True) for t in (u, X, W_V))
    scale = 1.0 / math.sqrt(case.D_H)
    O = target_attn_inner(ud, Xd, Wd, cq, ck, scale, qi, ki, validate=False)
    O.backward(dO)
    torch.cuda.synchronize()
    hu, hX, hW, hdO = (_host(t) for t in (u, X, W_V, dO))
    cq_h, ck_h = _cu_np(case.q_lens), _cu_np(case.k_lens)
    # float64 for the fp32 path (its own fp32 rounding is what is measured)
    odt = np.float64 if dtype == torch.float32 else np.float32
    O_r, _ = oa.forward(hu, hX, hW, cq_h, ck_h, scale, odt)
    du_r, dX_r, dW_r = oa.backward(hu, hX, hW, hdO, cq_h, ck_h, scale, odt)
    for n, a, r in (("O", O, O_r), ("du", ud.grad, du_r), ("dX", Xd.grad, dX_r),
                    ("dW_V", Wd.grad, dW_r)):
        assert_close(n, a, r)


def test_c5_full_plan_forward(device):
    case = W.config5(seed=0)
    lq, lk = np.asarray(case.q_lens), np.asarray(case.k_lens)
    capped = np.flatnonzero(lk == lk.max())
    capped = capped[np.argsort(-lq[capped], kind="stable")][:56]
    pick = np.unique(np.concatenate([np.arange(200), capped]))
    print(f"[C5 full] samples={len(lq)} T_q={int(lq.sum())} T_k={int(lk.sum())}; "
          f"checking {len(pick)} samples ({len(capped)} at Lk={int(lk.max())})", flush=True)
    u, X, W_V = _absorb_inputs(case, device)
    cq, ck = W.cu_from_lens(case.q_lens, device), W.cu_from_lens(case.k_lens, device)
    qi, ki = prepare_target_attn_indices(cq, ck)
    scale = 1.0 / math.sqrt(case.D_H)
    with torch.no_grad():
        O = target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)
    torch.cuda.synchronize()
    cq_h, ck_h = _cu_np(case.q_lens), _cu_np(case.k_lens)
    q_rows = np.concatenate([np.arange(cq_h[i], cq_h[i + 1]) for i in pick])
    k_rows = np.concatenate([np.arange(ck_h[i], ck_h[i + 1]) for i in pick])
    qr, kr = torch.from_numpy(q_rows).to(device), torch.from_numpy(k_rows).to(device)
    O_r, _ = oa.forward(_host(u[qr]), _host(X[kr]), _host(W_V), _cu_np(lq[pick]),
                        _cu_np(lk[pick]), scale, np.float32)
    assert_close("O", O[qr], O_r)
