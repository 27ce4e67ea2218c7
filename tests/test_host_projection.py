"""The host-side u projection of packed_target_attn (CPU, float64).

u[t,h,:] = (q_raw[t] W_Q[:,h,:]) W_K[:,h,:]^T (ta/interface.py:434-435) is
built as one GEMM against a block-diagonal matrix with a hand-written
per-head backward; both are checked against torch autograd through the
reference's two-einsum formulation.
"""
import torch

from varlenabsorbflashattn_amd.absorb import _project_u


def _reference(q_raw, W_Q, W_K):
    q_proj = torch.einsum("td,dhk->thk", q_raw, W_Q)
    return torch.einsum("thk,jhk->thj", q_proj, W_K)


def _inputs(T, d_q, d_kv, H, D_H, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64).requires_grad_(True)
    return mk(T, d_q), mk(d_q, H, D_H), mk(d_kv, H, D_H), g


def test_projection_values_layout_and_grads():
    for (T, d_q, d_kv, H, D_H) in [(37, 20, 11, 3, 5), (1, 8, 8, 1, 4), (64, 48, 40, 8, 4)]:
        q_raw, W_Q, W_K, g = _inputs(T, d_q, d_kv, H, D_H, seed=T + H)
        u = _project_u(q_raw, W_Q, W_K)
        u_ref = _reference(q_raw, W_Q, W_K)
        assert u.shape == (T, H, d_kv) and u.is_contiguous()
        torch.testing.assert_close(u, u_ref, rtol=1e-12, atol=1e-12)
        du = torch.randn(T, H, d_kv, generator=g, dtype=torch.float64)
        got = torch.autograd.grad(u, (q_raw, W_Q, W_K), du)
        want = torch.autograd.grad(u_ref, (q_raw, W_Q, W_K), du)
        for a, b in zip(got, want):
            torch.testing.assert_close(a, b, rtol=1e-11, atol=1e-11)


def test_projection_heads_do_not_mix():
    # one head's W_K zeroed: exactly that head's u columns vanish, and a
    # gradient on one head reaches only that head's slice of W_K
    q_raw, W_Q, W_K, g = _inputs(9, 6, 7, 4, 3, seed=5)
    with torch.no_grad():
        W_K[:, 2, :] = 0
    u = _project_u(q_raw, W_Q, W_K)
    assert torch.count_nonzero(u[:, 2, :]) == 0
    assert torch.count_nonzero(u[:, [0, 1, 3], :]) == u[:, [0, 1, 3], :].numel()
    du = torch.zeros_like(u)
    du[:, 1, :] = 1.0
    (dW_K,) = torch.autograd.grad(u, (W_K,), du)
    assert torch.count_nonzero(dW_K[:, [0, 2, 3], :]) == 0
    assert torch.count_nonzero(dW_K[:, 1, :]) == dW_K[:, 1, :].numel()
