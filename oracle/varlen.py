"""Block-diagonal (packed varlen) attention, numpy restatement (test oracle only).

Follows the reference's fp32 oracles: fa/test_smoke.py:29-70 (forward,
per segment, per head, explicit matmul -> softmax -> matmul) and
fa/test_smoke.py:73-164 (segmented backward).  The backward here is the
closed-form softmax-attention gradient (dV = P^T dO, dP = dO V^T,
dS = P*(dP - rowsum(P*dP)), dQ = scale dS K, dK = scale dS^T Q); the tests
pin it against torch.autograd on a float64 restatement and against finite
differences.

Conventions kept from the reference kernels (fa/kernels.py:24-35):
  * q/k/v/o are token-major ``[T, H, D]``;
  * LSE is ``[T_q, H]`` in the log2 domain: ``lse = log2(sum_j exp(scale*s_j))``.
Segments with Lq>0 and Lk==0 produce O=0 and LSE=-inf (the reference
oracle at fa/test_smoke.py:29-70 yields 0 there; the reference kernel's
division by zero is not reproduced).
"""
from __future__ import annotations

import numpy as np

LOG2E = 1.4426950408889634


def _segs(cu_q, cu_k):
    cq = np.asarray(cu_q, dtype=np.int64)
    ck = np.asarray(cu_k, dtype=np.int64)
    assert cq.shape == ck.shape
    for i in range(cq.size - 1):
        yield int(cq[i]), int(cq[i + 1]), int(ck[i]), int(ck[i + 1])


def forward(q, k, v, cu_q, cu_k, scale, dtype=np.float32):
    """Returns ``(o [T_q,H,D], lse [T_q,H] log2-domain)`` in ``dtype``."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    T_q, H, D = q.shape
    o = np.zeros((T_q, H, D), dtype=dtype)
    lse = np.full((T_q, H), -np.inf, dtype=dtype)
    for q0, q1, k0, k1 in _segs(cu_q, cu_k):
        if q1 == q0 or k1 == k0:
            continue
        qh = q[q0:q1].transpose(1, 0, 2)            # [H, Lq, D]
        kh = k[k0:k1].transpose(1, 0, 2)            # [H, Lk, D]
        vh = v[k0:k1].transpose(1, 0, 2)
        s = np.matmul(qh, kh.transpose(0, 2, 1)) * dtype(scale)   # [H, Lq, Lk]
        m = s.max(axis=-1, keepdims=True)
        e = np.exp(s - m)
        l = e.sum(axis=-1, keepdims=True)
        p = e / l
        o[q0:q1] = np.matmul(p, vh).transpose(1, 0, 2)
        lse[q0:q1] = ((m[..., 0] + np.log(l[..., 0])) * dtype(LOG2E)).T
    return o, lse


def backward(q, k, v, do, cu_q, cu_k, scale, dtype=np.float32, round_ps=None):
    """Returns ``(dq, dk, dv)`` (same shapes as q, k, v) in ``dtype``.

    ``round_ps`` (a function of an array, e.g. rounding to bf16) applies the
    reference kernels' rounding points: delta = rowsum(O * dO) is formed from
    O as stored in the input dtype (fa/kernels.py:186-216 reads the forward's
    output), P is rounded before dV = P^T dO and dS before dQ = dS K and
    dK = dS^T Q (fa/kernels.py:345, 480, 489).  With None every step is exact
    in ``dtype``."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    do = np.asarray(do, dtype=dtype)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    sc = dtype(scale)
    for q0, q1, k0, k1 in _segs(cu_q, cu_k):
        if q1 == q0 or k1 == k0:
            continue
        qh = q[q0:q1].transpose(1, 0, 2)
        kh = k[k0:k1].transpose(1, 0, 2)
        vh = v[k0:k1].transpose(1, 0, 2)
        doh = do[q0:q1].transpose(1, 0, 2)          # [H, Lq, D]
        s = np.matmul(qh, kh.transpose(0, 2, 1)) * sc
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        dvh = np.matmul(p.transpose(0, 2, 1), doh)              # [H, Lk, D]
        dp = np.matmul(doh, vh.transpose(0, 2, 1))              # [H, Lq, Lk]
        if round_ps is None:
            delta = (p * dp).sum(axis=-1, keepdims=True)
        else:
            o_r = np.asarray(round_ps(np.matmul(p, vh)), dtype=dtype)      # [H, Lq, D]
            delta = (o_r * doh).sum(axis=-1, keepdims=True)
        ds = p * (dp - delta)
        if round_ps is not None:
            dvh = np.matmul(np.asarray(round_ps(p), dtype=dtype).transpose(0, 2, 1), doh)
            ds = np.asarray(round_ps(ds), dtype=dtype)
        dq[q0:q1] = (np.matmul(ds, kh) * sc).transpose(1, 0, 2)
        dk[k0:k1] = (np.matmul(ds.transpose(0, 2, 1), qh) * sc).transpose(1, 0, 2)
        dv[k0:k1] = dvh.transpose(1, 0, 2)
    return dq, dk, dv


def combine(partial_o, partial_lse):
    """LSE merge of split-K partials (fa/kernels.py:639-647).

    ``partial_o [S, ..., D]`` normalized per split, ``partial_lse [S, ...]``
    log2 domain (-inf for an empty split).  Returns ``(o, lse)``.
    """
    po = np.asarray(partial_o, dtype=np.float64)
    pl = np.asarray(partial_lse, dtype=np.float64)
    m = pl.max(axis=0)
    m_safe = np.where(np.isneginf(m), 0.0, m)
    w = np.exp2(pl - m_safe)
    l = w.sum(axis=0)
    l_safe = np.where(l == 0, 1.0, l)
    o = (po * w[..., None]).sum(axis=0) / l_safe[..., None]
    lse = np.where(np.isneginf(m), -np.inf, m_safe + np.log2(l_safe))
    return o, lse
