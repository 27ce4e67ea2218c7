"""Pins of the CPU oracle (CPU only).

Each oracle function is checked against something independent of its own
formula: closed forms, torch.autograd on a float64 restatement, central
finite differences and the explicit-K/V formulation of absorb attention.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from conftest import ROOT
from oracle import absorb as oa
from oracle import varlen as ov

LN2 = math.log(2.0)


def _cu(lens):
    c = np.zeros(len(lens) + 1, dtype=np.int64)
    c[1:] = np.cumsum(lens)
    return c


def _rand(rng, *shape):
    return rng.standard_normal(shape)


# ---- varlen forward -----------------------------------------------------------

def test_zero_query_gives_segment_mean_and_log_length():
    rng = np.random.default_rng(0)
    lq, lk, H, D = [3, 5], [7, 2], 2, 8
    q = np.zeros((8, H, D))
    k, v = _rand(rng, 9, H, D), _rand(rng, 9, H, D)
    o, lse = ov.forward(q, k, v, _cu(lq), _cu(lk), 0.3, np.float64)
    np.testing.assert_allclose(o[:3], np.broadcast_to(v[:7].mean(0), (3, H, D)), atol=1e-12)
    np.testing.assert_allclose(o[3:], np.broadcast_to(v[7:].mean(0), (5, H, D)), atol=1e-12)
    np.testing.assert_allclose(lse[:3], math.log2(7), atol=1e-12)
    np.testing.assert_allclose(lse[3:], math.log2(2), atol=1e-12)


def test_single_key_returns_value():
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 4, 2, 16), _rand(rng, 1, 2, 16), _rand(rng, 1, 2, 16)
    o, _ = ov.forward(q, k, v, _cu([4]), _cu([1]), 0.25, np.float64)
    np.testing.assert_allclose(o, np.broadcast_to(v, o.shape), atol=1e-12)


def test_empty_key_segment_gives_zero_and_neg_inf():
    rng = np.random.default_rng(2)
    q, k, v = _rand(rng, 3, 1, 8), _rand(rng, 4, 1, 8), _rand(rng, 4, 1, 8)
    o, lse = ov.forward(q, k, v, _cu([2, 1]), _cu([0, 4]), 0.3, np.float64)
    assert (o[:2] == 0).all() and np.isneginf(lse[:2]).all() and np.isfinite(lse[2:]).all()


def test_one_hot_segment_values_pin_masking():
    rng = np.random.default_rng(3)
    lens = [3, 9, 1, 14]
    T, H, D = sum(lens), 2, 8
    seg = np.repeat(np.arange(len(lens)), lens)
    v = np.zeros((T, H, D))
    v[np.arange(T), :, seg] = 1.0
    o, _ = ov.forward(_rand(rng, T, H, D), _rand(rng, T, H, D), v, _cu(lens), _cu(lens), 0.4,
                      np.float64)
    want = np.zeros_like(o)
    want[np.arange(T), :, seg] = 1.0
    np.testing.assert_allclose(o, want, atol=1e-12)


def test_forward_matches_torch_and_scipy_logsumexp():
    from scipy.special import logsumexp
    rng = np.random.default_rng(4)
    lq, lk, H, D, sc = [5, 0, 11], [6, 3, 17], 3, 16, 0.37
    q, k, v = _rand(rng, 16, H, D), _rand(rng, 26, H, D), _rand(rng, 26, H, D)
    o, lse = ov.forward(q, k, v, _cu(lq), _cu(lk), sc, np.float64)
    cq, ck = _cu(lq), _cu(lk)
    for s in range(3):
        if lq[s] == 0:
            continue
        qs = torch.from_numpy(q[cq[s]:cq[s + 1]]).transpose(0, 1)
        ks = torch.from_numpy(k[ck[s]:ck[s + 1]]).transpose(0, 1)
        vs = torch.from_numpy(v[ck[s]:ck[s + 1]]).transpose(0, 1)
        sco = (qs @ ks.transpose(1, 2)) * sc
        ref = (torch.softmax(sco, -1) @ vs).transpose(0, 1).numpy()
        np.testing.assert_allclose(o[cq[s]:cq[s + 1]], ref, atol=1e-12)
        np.testing.assert_allclose(lse[cq[s]:cq[s + 1]].T, logsumexp(sco.numpy(), -1) / LN2,
                                   atol=1e-12)


def test_combine_identity_on_key_splits():
    rng = np.random.default_rng(5)
    Lq, Lk, H, D, sc = 6, 50, 2, 8, 0.5
    q, k, v = _rand(rng, Lq, H, D), _rand(rng, Lk, H, D), _rand(rng, Lk, H, D)
    full_o, full_lse = ov.forward(q, k, v, _cu([Lq]), _cu([Lk]), sc, np.float64)
    bounds = [0, 7, 7, 30, 50]  # includes an empty split
    parts = [ov.forward(q, k[a:b], v[a:b], _cu([Lq]), _cu([b - a]), sc, np.float64)
             for a, b in zip(bounds, bounds[1:])]
    o, lse = ov.combine(np.stack([p[0] for p in parts]), np.stack([p[1] for p in parts]))
    np.testing.assert_allclose(o, full_o, atol=1e-12)
    np.testing.assert_allclose(lse, full_lse, atol=1e-12)


# ---- varlen backward ----------------------------------------------------------

def _torch_varlen(q, k, v, lq, lk, sc):
    cq, ck = _cu(lq), _cu(lk)
    outs = []
    for s in range(len(lq)):
        qs, ks, vs = q[cq[s]:cq[s + 1]], k[ck[s]:ck[s + 1]], v[ck[s]:ck[s + 1]]
        if qs.shape[0] == 0:
            continue
        if ks.shape[0] == 0:
            outs.append(torch.zeros_like(qs))
            continue
        p = torch.softmax(torch.einsum("qhd,khd->hqk", qs, ks) * sc, -1)
        outs.append(torch.einsum("hqk,khd->qhd", p, vs))
    return torch.cat(outs)


def test_backward_matches_torch_autograd():
    rng = np.random.default_rng(6)
    lq, lk, H, D, sc = [4, 9, 0, 3], [5, 12, 2, 0], 2, 8, 0.35
    q, k, v = _rand(rng, 16, H, D), _rand(rng, 19, H, D), _rand(rng, 19, H, D)
    do = _rand(rng, 16, H, D)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    _torch_varlen(tq, tk, tv, lq, lk, sc).backward(torch.from_numpy(do))
    dq, dk, dv = ov.backward(q, k, v, do, _cu(lq), _cu(lk), sc, np.float64)
    for a, b in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        np.testing.assert_allclose(a, b.numpy(), atol=1e-10)


def test_backward_finite_differences():
    rng = np.random.default_rng(7)
    lq, lk, H, D, sc = [3, 2], [4, 3], 1, 4, 0.7
    q, k, v = _rand(rng, 5, H, D), _rand(rng, 7, H, D), _rand(rng, 7, H, D)
    do = _rand(rng, 5, H, D)
    dq, dk, dv = ov.backward(q, k, v, do, _cu(lq), _cu(lk), sc, np.float64)

    def loss(q_, k_, v_):
        return float((ov.forward(q_, k_, v_, _cu(lq), _cu(lk), sc, np.float64)[0] * do).sum())

    eps = 1e-6
    for arr, grad, pos in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        for idx in [(0, 0, 1), (arr.shape[0] - 1, 0, 3), (2, 0, 2)]:
            args = [q.copy(), k.copy(), v.copy()]
            args[pos][idx] += eps
            lp = loss(*args)
            args[pos][idx] -= 2 * eps
            lm = loss(*args)
            assert abs((lp - lm) / (2 * eps) - grad[idx]) < 1e-6


def _brute_backward_rounded(q, k, v, do, lq, lk, sc, r):
    """Scalar loops over one head: softmax attention backward with the
    rounding ``r`` applied to each P and dS element before the products that
    consume them (dV = r(P)^T dO, dQ = sc r(dS) K, dK = sc r(dS)^T Q) and to
    O before delta = O . dO."""
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    q0 = k0 = 0
    D = q.shape[-1]
    for a, b in zip(lq, lk):
        for h in range(q.shape[1]):
            for i in range(q0, q0 + a):
                s = [sc * sum(q[i, h, d] * k[j, h, d] for d in range(D)) for j in range(k0, k0 + b)]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                p = [x / sum(e) for x in e]
                dp = [sum(do[i, h, d] * v[j, h, d] for d in range(D)) for j in range(k0, k0 + b)]
                o = [r(sum(pp * v[j, h, d] for pp, j in zip(p, range(k0, k0 + b))))
                     for d in range(D)]
                delta = sum(o[d] * do[i, h, d] for d in range(D))
                for jj, j in enumerate(range(k0, k0 + b)):
                    ds = r(p[jj] * (dp[jj] - delta))
                    for d in range(D):
                        dv[j, h, d] += r(p[jj]) * do[i, h, d]
                        dq[i, h, d] += sc * ds * k[j, h, d]
                        dk[j, h, d] += sc * ds * q[i, h, d]
        q0 += a
        k0 += b
    return dq, dk, dv


def test_backward_reference_rounding_points():
    """round_ps applies the reference kernels' roundings of P (before dV) and
    dS (before dQ and dK): pinned against scalar loops with a coarse rounding
    (two decimals, so a rounding applied to the wrong product or missing
    shows), the identity rounding reproduces the exact backward (to the
    summation order of delta = O . dO against sum_j P dP), and every gradient
    moves under the coarse rounding."""
    rng = np.random.default_rng(8)
    lq, lk, H, D, sc = [3, 2, 0], [4, 3, 2], 2, 3, 0.9
    q, k, v = _rand(rng, 5, H, D), _rand(rng, 9, H, D), _rand(rng, 9, H, D)
    do = _rand(rng, 5, H, D)
    coarse = lambda x: np.round(x, 2)
    got = ov.backward(q, k, v, do, _cu(lq), _cu(lk), sc, np.float64, round_ps=coarse)
    want = _brute_backward_rounded(q, k, v, do, lq, lk, sc, lambda x: round(x, 2))
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, atol=1e-12)
    exact = ov.backward(q, k, v, do, _cu(lq), _cu(lk), sc, np.float64)
    same = ov.backward(q, k, v, do, _cu(lq), _cu(lk), sc, np.float64, round_ps=lambda x: x)
    for a, b, c in zip(exact, same, got):
        np.testing.assert_allclose(a, b, atol=1e-12)  # delta summed in another order
        assert np.abs(a - c).max() > 1e-4


# ---- absorb ---------------------------------------------------------------------

def _absorb_inputs(rng, lq, lk, d_q=12, d_kv=10, H=2, D_H=4):
    return (_rand(rng, sum(lq), d_q) * 0.5, _rand(rng, sum(lk), d_kv) * 0.5,
            _rand(rng, d_q, H, D_H) * 0.5, _rand(rng, d_kv, H, D_H) * 0.5,
            _rand(rng, d_kv, H, D_H) * 0.5)


def _brute_absorb_backward_rounded(q_raw, X, W_Q, W_K, W_V, dO, lq, lk, sc, r):
    """Scalar loops: grads of the absorbed op with the rounding ``r`` at each
    rounding point the reference's kernels and 16-bit products have (q_proj,
    u, dAX, P, dS, aX, du, dq_proj, and O before delta = O . dO)."""
    T, d_q = q_raw.shape
    F, H, DH = W_K.shape
    qp = np.zeros((T, H, DH))
    u = np.zeros((T, H, F))
    for t in range(T):
        for h in range(H):
            for d in range(DH):
                qp[t, h, d] = r(sum(q_raw[t, c] * W_Q[c, h, d] for c in range(d_q)))
            for f in range(F):
                u[t, h, f] = r(sum(qp[t, h, d] * W_K[f, h, d] for d in range(DH)))
    du, dX, ax = np.zeros_like(u), np.zeros_like(X), np.zeros_like(u)
    dax = np.zeros_like(u)
    for t in range(T):
        for h in range(H):
            for f in range(F):
                dax[t, h, f] = r(sum(dO[t, h, d] * W_V[f, h, d] for d in range(DH)))
    q0 = k0 = 0
    for a, b in zip(lq, lk):
        for t in range(q0, q0 + a):
            for h in range(H):
                s = [sc * sum(u[t, h, f] * X[j, f] for f in range(F)) for j in range(k0, k0 + b)]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                p = [x / sum(e) for x in e]
                dp = [sum(dax[t, h, f] * X[j, f] for f in range(F)) for j in range(k0, k0 + b)]
                axr = [sum(pp * X[j, f] for pp, j in zip(p, range(k0, k0 + b))) for f in range(F)]
                o = [r(sum(axr[f] * W_V[f, h, d] for f in range(F))) for d in range(DH)]
                delta = sum(o[d] * dO[t, h, d] for d in range(DH))
                for jj, j in enumerate(range(k0, k0 + b)):
                    ds, pr = r(p[jj] * (dp[jj] - delta)), r(p[jj])
                    for f in range(F):
                        ax[t, h, f] += pr * X[j, f]
                        du[t, h, f] += sc * ds * X[j, f]
                        dX[j, f] += sc * ds * u[t, h, f] + pr * dax[t, h, f]
        q0 += a
        k0 += b
    dW_V = np.zeros_like(W_V)
    dqp, dW_K, dW_Q, dq = np.zeros_like(qp), np.zeros_like(W_K), np.zeros_like(W_Q), np.zeros_like(q_raw)
    for t in range(T):
        for h in range(H):
            for f in range(F):
                du[t, h, f] = r(du[t, h, f])
                for d in range(DH):
                    dW_V[f, h, d] += r(ax[t, h, f]) * dO[t, h, d]
            for d in range(DH):
                dqp[t, h, d] = r(sum(du[t, h, f] * W_K[f, h, d] for f in range(F)))
    for t in range(T):
        for h in range(H):
            for d in range(DH):
                for f in range(F):
                    dW_K[f, h, d] += du[t, h, f] * qp[t, h, d]
                for c in range(d_q):
                    dW_Q[c, h, d] += q_raw[t, c] * dqp[t, h, d]
                    dq[t, c] += dqp[t, h, d] * W_Q[c, h, d]
    return dq, dX, dW_Q, dW_K, dW_V


def test_absorb_backward_reference_rounding_points():
    """full_backward(round_to=...) applies the reference's rounding points:
    pinned against scalar loops with a coarse rounding (two decimals, so a
    rounding missing or applied to the wrong operand shows); the identity
    rounding reproduces the exact gradients (to the summation order of delta
    = O . dO against sum_j P dP), and every gradient moves under the coarse
    rounding."""
    rng = np.random.default_rng(9)
    lq, lk = [2, 1, 0], [3, 2, 4]
    ins = _absorb_inputs(rng, lq, lk, d_q=3, d_kv=3, H=2, D_H=2)
    ins = tuple(x * 3 for x in ins)
    dO = _rand(rng, sum(lq), 2, 2)
    sc, cu_q, cu_k = 0.8, _cu(lq), _cu(lk)
    got = oa.full_backward(*ins, dO, cu_q, cu_k, sc, np.float64, round_to=lambda x: np.round(x, 2))
    want = _brute_absorb_backward_rounded(*ins, dO, lq, lk, sc, lambda x: round(x, 2))
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, atol=1e-10)
    exact = oa.full_backward(*ins, dO, cu_q, cu_k, sc, np.float64)
    same = oa.full_backward(*ins, dO, cu_q, cu_k, sc, np.float64, round_to=lambda x: x)
    for a, b, c in zip(exact, same, got):
        np.testing.assert_allclose(a, b, atol=1e-12)
        assert np.abs(a - c).max() > 1e-4


def test_absorbed_equals_explicit():
    rng = np.random.default_rng(8)
    lq, lk = [3, 1, 4], [5, 2, 9]
    ins = _absorb_inputs(rng, lq, lk)
    a = oa.full_forward(*ins, _cu(lq), _cu(lk), 0.5, np.float64)
    b = oa.explicit_forward(*ins, _cu(lq), _cu(lk), 0.5, np.float64)
    np.testing.assert_allclose(a, b, atol=1e-12)


def test_absorb_backward_matches_torch_autograd():
    rng = np.random.default_rng(9)
    lq, lk, sc = [3, 1, 0, 4], [5, 2, 3, 9], 0.5
    ins = _absorb_inputs(rng, lq, lk)
    dO = _rand(rng, sum(lq), 2, 4)
    t = [torch.tensor(x, requires_grad=True) for x in ins]
    q_raw, X, W_Q, W_K, W_V = t
    cq, ck = _cu(lq), _cu(lk)
    outs = []
    for s in range(len(lq)):
        qs, xs = q_raw[cq[s]:cq[s + 1]], X[ck[s]:ck[s + 1]]
        if qs.shape[0] == 0:
            continue
        K = torch.einsum("ka,ahd->khd", xs, W_K)
        V = torch.einsum("ka,ahd->khd", xs, W_V)
        Q = torch.einsum("qa,ahd->qhd", qs, W_Q)
        p = torch.softmax(torch.einsum("qhd,khd->hqk", Q, K) * sc, -1)
        outs.append(torch.einsum("hqk,khd->qhd", p, V))
    torch.cat(outs).backward(torch.from_numpy(dO))
    grads = oa.full_backward(*ins, dO, cq, ck, sc, np.float64)
    for g, tt in zip(grads, t):
        np.testing.assert_allclose(g, tt.grad.numpy(), atol=1e-10)


def test_absorb_inner_lse_and_uniform_case():
    rng = np.random.default_rng(10)
    lq, lk = [2, 3], [4, 6]
    u = np.zeros((5, 2, 10))
    X = _rand(rng, 10, 10)
    W_V = _rand(rng, 10, 2, 4)
    O, lse = oa.forward(u, X, W_V, _cu(lq), _cu(lk), 0.5, np.float64)
    want0 = X[:4].mean(0) @ W_V[:, 0, :]
    np.testing.assert_allclose(O[0, 0], want0, atol=1e-12)
    np.testing.assert_allclose(lse[:2], math.log2(4), atol=1e-12)
    np.testing.assert_allclose(lse[2:], math.log2(6), atol=1e-12)


# ---- committed golden summary of configs[0] --------------------------------------

def test_config1_golden_summary():
    path = os.path.join(ROOT, "tests", "golden", "config1_oracle_summary.json")
    gold = json.load(open(path))
    from tests.golden.make_golden import config1_outputs, summarize
    outs = config1_outputs()
    for name, arr in outs.items():
        s = summarize(arr)
        for key in ("sum", "abs_sum", "samples"):
            np.testing.assert_allclose(s[key], gold[name][key], rtol=1e-9, atol=1e-9)
