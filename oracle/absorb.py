"""Absorbed ragged target attention, numpy restatement (test oracle only).

Math (ta/kernels.py:23-45, ta/interface.py:429-435):
  u[t,h,:]  = (q_raw[t] @ W_Q[:,h,:]) @ W_K[:,h,:]^T          [T_q, H, D_KV]
  S[t,h,j]  = scale * u[t,h,:] . X[j,:]       (j in the segment of t)
  P         = softmax_j(S)
  aX[t,h,:] = sum_j P[t,h,j] X[j,:]
  O[t,h,:]  = aX[t,h,:] @ W_V[:,h,:]                            [T_q, H, D_H]

Restates ta/test_smoke.py:188-229 (absorbed) and ta/test_smoke.py:111-147 /
150-185 (explicit K = X W_K, V = X W_V) in fp32 (or float64) without the
reference oracles' rounding of p to the input dtype.  Gradients are the
closed forms (dAX = dO W_V^T, dP = dAX X^T, dS = P*(dP - rowsum(P*dP)),
du = scale dS X, dX = scale dS^T u + P^T dAX, dW_V = aX^T dO); tests pin
them against torch.autograd on a float64 restatement.

LSE is ``[T_q, H]`` log2 domain (ta/kernels.py:18-21); empty-key segments
give O=0, LSE=-inf.
"""
from __future__ import annotations

import numpy as np

LOG2E = 1.4426950408889634


def _segs(cu_q, cu_k):
    cq = np.asarray(cu_q, dtype=np.int64)
    ck = np.asarray(cu_k, dtype=np.int64)
    for i in range(cq.size - 1):
        yield int(cq[i]), int(cq[i + 1]), int(ck[i]), int(ck[i + 1])


def project_u(q_raw, W_Q, W_K, dtype=np.float32):
    """u = q_raw @ W_Q @ W_K^T per head (ta/interface.py:434-435)."""
    q_raw = np.asarray(q_raw, dtype=dtype)
    W_Q = np.asarray(W_Q, dtype=dtype)
    W_K = np.asarray(W_K, dtype=dtype)
    T, d_q = q_raw.shape
    _, H, D_H = W_Q.shape
    qp = (q_raw @ W_Q.reshape(d_q, H * D_H)).reshape(T, H, D_H)
    return np.einsum("thd,khd->thk", qp, W_K)


def _per_head(a, W):
    """einsum('thf,fhd->thd', a, W) as one 2-D product per head."""
    T, H, _ = a.shape
    out = np.empty((T, H, W.shape[2]), dtype=np.result_type(a, W))
    for h in range(H):
        out[:, h, :] = a[:, h, :] @ W[:, h, :]
    return out


def forward(u, X, W_V, cu_q, cu_k, scale, dtype=np.float32, return_ax=False):
    """Inner op: returns ``(O [T_q,H,D_H], lse [T_q,H])`` (and aX if asked).

    Per segment the (token, head) rows are one ``[Lq*H, D_KV]`` matrix, so
    scores and P.X are plain 2-D products against the segment's X rows.
    """
    u = np.asarray(u, dtype=dtype)
    X = np.asarray(X, dtype=dtype)
    W_V = np.asarray(W_V, dtype=dtype)
    T_q, H, D_KV = u.shape
    ax = np.zeros((T_q, H, D_KV), dtype=dtype)
    lse = np.full((T_q, H), -np.inf, dtype=dtype)
    for q0, q1, k0, k1 in _segs(cu_q, cu_k):
        if q1 == q0 or k1 == k0:
            continue
        xs = X[k0:k1]
        s = (u[q0:q1].reshape(-1, D_KV) @ xs.T) * dtype(scale)      # [Lq*H, Lk]
        m = s.max(axis=-1, keepdims=True)
        e = np.exp(s - m)
        l = e.sum(axis=-1, keepdims=True)
        ax[q0:q1] = ((e / l) @ xs).reshape(q1 - q0, H, D_KV)
        lse[q0:q1] = ((m[:, 0] + np.log(l[:, 0])) * dtype(LOG2E)).reshape(q1 - q0, H)
    O = _per_head(ax, W_V).astype(dtype)
    if return_ax:
        return O, lse, ax
    return O, lse


def _ident(x):
    return x


def backward(u, X, W_V, dO, cu_q, cu_k, scale, dtype=np.float32, round_to=None):
    """Inner op backward: returns ``(du, dX, dW_V)``.

    ``round_to`` (a function of an array, e.g. rounding to bf16) applies the
    reference kernels' rounding points: delta = rowsum(O * dO) from O as
    stored in the input dtype (ta/kernels.py:298-325 reads the forward's
    output), dAX = dO W_V^T before the products it feeds (ta/kernels.py:480,
    and the dX kernels), P and dS before the products with X and u (484-486),
    aX before dW_V = aX^T dO (491), and du on its store (498).  With None
    every step is exact in ``dtype``."""
    r = _ident if round_to is None else (lambda a: np.asarray(round_to(a), dtype=dtype))
    u = np.asarray(u, dtype=dtype)
    X = np.asarray(X, dtype=dtype)
    W_V = np.asarray(W_V, dtype=dtype)
    dO = np.asarray(dO, dtype=dtype)
    T_q, H, D_KV = u.shape
    sc = dtype(scale)
    du = np.zeros_like(u)
    dX = np.zeros_like(X)
    ax_all = np.zeros_like(u)
    dax_all = np.empty_like(u)                                   # dO W_V^T per head
    for h in range(H):
        dax_all[:, h, :] = dO[:, h, :] @ W_V[:, h, :].T
    dax_all = r(dax_all)
    for q0, q1, k0, k1 in _segs(cu_q, cu_k):
        if q1 == q0 or k1 == k0:
            continue
        xs = X[k0:k1]
        u2 = u[q0:q1].reshape(-1, D_KV)                          # [Lq*H, D_KV]
        dax = dax_all[q0:q1].reshape(-1, D_KV)
        s = (u2 @ xs.T) * sc
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)                       # [Lq*H, Lk]
        dp = dax @ xs.T
        if round_to is None:
            delta = (p * dp).sum(axis=-1, keepdims=True)
        else:  # O = (P X) W_V per head, rounded, dotted with dO
            o_r = r(_per_head((p @ xs).reshape(q1 - q0, H, D_KV), W_V))
            delta = (o_r * dO[q0:q1]).sum(axis=-1).reshape(-1, 1)
        ds = r(p * (dp - delta))
        p = r(p)
        ax_all[q0:q1] = (p @ xs).reshape(q1 - q0, H, D_KV)
        du[q0:q1] = ((ds @ xs) * sc).reshape(q1 - q0, H, D_KV)
        dX[k0:k1] = (ds.T @ u2) * sc + p.T @ dax
    ax_all = r(ax_all)
    dW_V = np.empty_like(W_V)
    for h in range(H):
        dW_V[:, h, :] = ax_all[:, h, :].T @ dO[:, h, :]
    return r(du), dX, dW_V


def full_forward(q_raw, X, W_Q, W_K, W_V, cu_q, cu_k, scale, dtype=np.float32):
    """``packed_target_attn`` forward: O [T_q, H, D_H]."""
    u = project_u(q_raw, W_Q, W_K, dtype)
    return forward(u, X, W_V, cu_q, cu_k, scale, dtype)[0]


def full_backward(q_raw, X, W_Q, W_K, W_V, dO, cu_q, cu_k, scale, dtype=np.float32,
                  round_to=None):
    """Grads of ``packed_target_attn`` w.r.t. (q_raw, X, W_Q, W_K, W_V).

    The u-projection gradients follow the chain rule through
    ta/interface.py:434-435.  ``round_to`` applies, besides the inner
    backward's rounding points, those of the reference's 16-bit torch
    products: q_proj and u in the forward, dq_proj = du W_K before the
    products it feeds (dq_raw, dW_Q)."""
    r = _ident if round_to is None else (lambda a: np.asarray(round_to(a), dtype=dtype))
    q_raw = np.asarray(q_raw, dtype=dtype)
    W_Q = np.asarray(W_Q, dtype=dtype)
    W_K = np.asarray(W_K, dtype=dtype)
    T, d_q = q_raw.shape
    _, H, D_H = W_Q.shape
    qp = r((q_raw @ W_Q.reshape(d_q, H * D_H)).reshape(T, H, D_H))
    u = r(np.einsum("thd,khd->thk", qp, W_K))
    du, dX, dW_V = backward(u, X, W_V, dO, cu_q, cu_k, scale, dtype, round_to=round_to)
    dqp = r(np.einsum("thk,khd->thd", du, W_K))
    dW_K = np.einsum("thk,thd->khd", du, qp)
    dq_raw = dqp.reshape(T, H * D_H) @ W_Q.reshape(d_q, H * D_H).T
    dW_Q = (q_raw.T @ dqp.reshape(T, H * D_H)).reshape(d_q, H, D_H)
    return dq_raw, dX, dW_Q, dW_K, dW_V


def explicit_forward(q_raw, X, W_Q, W_K, W_V, cu_q, cu_k, scale, dtype=np.float64):
    """Explicit K = X W_K, V = X W_V per head (ta/test_smoke.py:111-147)."""
    q_raw = np.asarray(q_raw, dtype=dtype)
    X = np.asarray(X, dtype=dtype)
    W_Q, W_K, W_V = (np.asarray(w, dtype=dtype) for w in (W_Q, W_K, W_V))
    T_q = q_raw.shape[0]
    _, H, D_H = W_Q.shape
    O = np.zeros((T_q, H, D_H), dtype=dtype)
    for q0, q1, k0, k1 in _segs(cu_q, cu_k):
        if q1 == q0 or k1 == k0:
            continue
        for h in range(H):
            qp = q_raw[q0:q1] @ W_Q[:, h, :]
            kp = X[k0:k1] @ W_K[:, h, :]
            vp = X[k0:k1] @ W_V[:, h, :]
            s = qp @ kp.T * scale
            s -= s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            O[q0:q1, h, :] = p @ vp
    return O
