"""Ragged absorbed target attention -- drop-in for
``triton_target_attn_absorb`` (ta/interface.py:125-454).

``packed_target_attn`` keeps the reference signature.  For 16-bit inputs on
the matrix-core shapes it forms ``q_proj = q_raw W_Q`` and runs the attention
with ``u = q_proj W_K^T`` formed inside the attention kernel (u never reaches
memory in the forward); otherwise it projects ``u`` per head (this library's
projection kernels, or torch GEMMs for fp32 / odd widths, as in
ta/interface.py:429-435) and calls ``target_attn_inner``, whose forward and
backward run in ``libvafa.so``:
scores are taken directly against the raw ``X`` rows, ``aX = softmax(u X^T) X``
is accumulated on the fly and projected by ``W_V`` at the end.  The backward
is deterministic (dW_V and dX are reduced in a fixed order).
"""
from __future__ import annotations

import math
import os
import weakref
from typing import Optional

import numpy as np
import torch

from . import _lib

# Reference block sizes, kept for the (seg, block) tables that
# prepare_target_attn_indices returns (ta/interface.py:59-63).
_BT_Q_FWD = 16
_BT_K_BWD = 64

# prepare_target_attn_indices() remembers the host cu_seqlens behind the
# tables it returns, so a later validate=False call on the SAME, unmodified
# cu_seqlens tensors needs no device->host copy.  Keyed by id() of the query
# table with a weak reference to it; the cu_seqlens tensors are held by weak
# reference together with their version counters and data pointers, so any
# other pair of tensors (or an in-place change of these) takes the copy again.
_HOST_CU: dict = {}


def _cu_stamp(t):
    if not isinstance(t, torch.Tensor):
        return None
    return (weakref.ref(t), t._version, t.data_ptr())


def _stamp_matches(stamp, t) -> bool:
    if stamp is None or not isinstance(t, torch.Tensor):
        return False
    ref, version, data_ptr = stamp
    return ref() is t and t._version == version and t.data_ptr() == data_ptr


def _remember_host_cu(table: torch.Tensor, cu_q, cu_k, cu_q_h: np.ndarray,
                      cu_k_h: np.ndarray) -> None:
    key = id(table)
    _HOST_CU[key] = (weakref.ref(table, lambda _r, k=key: _HOST_CU.pop(k, None)),
                     _cu_stamp(cu_q), _cu_stamp(cu_k), cu_q_h, cu_k_h)


def _recall_host_cu(table: Optional[torch.Tensor], cu_q, cu_k):
    """Host copies taken when ``table`` was prepared, if ``cu_q`` / ``cu_k`` are
    the very tensors it was prepared from, unmodified since; else None."""
    if table is None:
        return None
    hit = _HOST_CU.get(id(table))
    if hit is None or hit[0]() is not table:
        return None
    if not (_stamp_matches(hit[1], cu_q) and _stamp_matches(hit[2], cu_k)):
        return None
    return hit[3], hit[4]


def _select_fwd_mode() -> str:
    """TRITON_TARGET_ATTN_FWD_MODE as in ta/interface.py:66-70.

    Both accepted modes run the same fused kernel here; the variable keeps
    its validation so existing configurations behave the same.
    """
    mode = os.environ.get("TRITON_TARGET_ATTN_FWD_MODE", "alpha").lower()
    if mode in ("direct", "alpha"):
        return mode
    raise ValueError("TRITON_TARGET_ATTN_FWD_MODE must be one of: direct, alpha")


def _select_dx_mode(n_k_chunks: int) -> str:
    """TRITON_TARGET_ATTN_DX_MODE as in ta/interface.py:73-85 (validation only:
    every mode maps to the deterministic dX kernel)."""
    mode = os.environ.get("TRITON_TARGET_ATTN_DX_MODE", "auto").lower()
    if mode in ("partial", "fused", "atomic"):
        return mode
    if mode != "auto":
        raise ValueError(
            "TRITON_TARGET_ATTN_DX_MODE must be one of: auto, partial, fused, atomic")
    return "fused" if n_k_chunks >= 1024 else "partial"


def _validate_cu_seqlens(cu_host: np.ndarray, shape, T: int, name: str) -> None:
    """ta/interface.py:92-106."""
    if len(shape) != 1 or cu_host.size < 2:
        raise ValueError(f"{name}: must be 1-D with len>=2, got {tuple(shape)}")
    _lib.validate_cu_absorb(cu_host, T, name)


def _next_power_of_2(x: int) -> int:
    if x < 1:
        raise ValueError(f"expected positive dimension, got {x}")
    return 1 << (x - 1).bit_length()


def prepare_target_attn_indices(cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor):
    """Chunk tables ``(q_idx [NT_q,2], k_idx [NT_k,2])`` (ta/interface.py:125-138).

    Same content as the reference (BT_Q=16, BT_K=64 rows ``(seg, block)``).
    Passing them back with ``validate=False`` together with the same
    cu_seqlens tensors skips every host round trip: the host cu_seqlens
    captured here are reused to look up the cached plan.  With other (or
    modified) cu_seqlens tensors the call copies them to the host again, so
    the plan always follows the cu_seqlens of the call, as the reference's
    kernels do (they read cu_seqlens on every call).
    """
    cu_q_h, cu_k_h = _lib.as_host_i64_pair(cu_seqlens_q, cu_seqlens_k)
    q_idx = torch.from_numpy(_lib.chunk_indices(cu_q_h, _BT_Q_FWD)).to(cu_seqlens_q.device)
    k_idx = torch.from_numpy(_lib.chunk_indices(cu_k_h, _BT_K_BWD)).to(cu_seqlens_k.device)
    _remember_host_cu(q_idx, cu_seqlens_q, cu_seqlens_k, cu_q_h, cu_k_h)
    return q_idx, k_idx


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 0), dtype=torch.uint8, device=device)


def _aligned(x: torch.Tensor) -> torch.Tensor:
    return x.clone() if x.data_ptr() % 16 != 0 else x


def _absorb_plan(T_q, T_k, H, D_KV, D_H, device, cu_seqlens_q, cu_seqlens_k,
                 q_chunk_indices, validate):
    """Validation (ta/interface.py:92-122, 176-201) and the cached device plan
    of one absorb call; host cu_seqlens come from the prepared index tables
    when they belong to these very tensors and validation is off."""
    known = _recall_host_cu(q_chunk_indices, cu_seqlens_q, cu_seqlens_k)
    if known is not None and not validate:
        cu_q_h, cu_k_h = known
    else:
        cu_q_h, cu_k_h = _lib.as_host_i64_pair(cu_seqlens_q, cu_seqlens_k)
    if validate:
        n_seg = cu_seqlens_q.numel() - 1
        assert cu_seqlens_k.numel() - 1 == n_seg, "segment count mismatch q vs k"
        _validate_cu_seqlens(cu_q_h, cu_seqlens_q.shape, T_q, "cu_seqlens_q")
        _validate_cu_seqlens(cu_k_h, cu_seqlens_k.shape, T_k, "cu_seqlens_k")
        _lib.check_active_have_keys(cu_q_h, cu_k_h)
    B_DKV = _next_power_of_2(D_KV)
    assert B_DKV <= 512, f"D_KV={D_KV} pads to {B_DKV}, which is too large for v1 tiles"
    plan = _lib.device_plan("absorb", cu_q_h, cu_k_h, (H, D_KV, D_H), device)
    if plan.info.T_q > T_q or plan.info.T_k > T_k:
        raise ValueError(
            f"cu_seqlens address {plan.info.T_q} query / {plan.info.T_k} key tokens but "
            f"the inputs hold {T_q} / {T_k}")
    if plan.info.n_fwd > 0:
        _select_fwd_mode()
    return plan


def _absorb_bwd(u, X, W_V, O, LSE, dO, plan, scale):
    """du, dX, dW_V of the inner op through vafa_absorb_bwd."""
    T_q, H, D_KV = u.shape
    D_H = W_V.shape[2]
    if dO.stride(-1) != 1 or not dO.is_contiguous():
        dO = dO.contiguous()
    if dO.dtype != u.dtype:
        dO = dO.to(u.dtype)
    dO = _aligned(dO)
    if plan.info.n_kv > 0:
        _select_dx_mode(int(plan.info.n_kv))
    du = torch.empty_like(u)
    dX = torch.empty_like(X)
    dW_V = torch.empty_like(W_V)
    L = _lib.lib()
    ws = _workspace(L.vafa_absorb_bwd_workspace(plan.info, D_KV, D_H), u.device)
    _lib.check(L.vafa_absorb_bwd(
        u.data_ptr(), X.data_ptr(), W_V.data_ptr(), O.data_ptr(), dO.data_ptr(),
        LSE.data_ptr(), du.data_ptr(), dX.data_ptr(), dW_V.data_ptr(),
        plan.items.data_ptr(), plan.info, D_KV, D_H, _lib.dtype_code(u.dtype),
        float(scale), ws.data_ptr() if ws.numel() else None, ws.numel(),
        _lib.stream_ptr(u.device)))
    return du, dX, dW_V


class _TargetAttnFunction(torch.autograd.Function):
    """Inner op on projected u (ta/interface.py:141-321)."""

    @staticmethod
    def forward(ctx, u, X, W_V, cu_seqlens_q, cu_seqlens_k, scale, q_chunk_indices,
                k_chunk_indices, validate):
        T_q, H, D_KV = u.shape
        T_k, D_KV_x = X.shape
        D_KV_wv, H_wv, D_H = W_V.shape
        assert D_KV == D_KV_x == D_KV_wv, \
            f"D_KV mismatch: u={D_KV}, X={D_KV_x}, W_V={D_KV_wv}"
        assert H == H_wv, f"H mismatch: u={H}, W_V={H_wv}"
        assert u.dtype == X.dtype == W_V.dtype, \
            f"u/X/W_V must share dtype, got {u.dtype}/{X.dtype}/{W_V.dtype}"
        assert u.is_cuda and X.is_cuda and W_V.is_cuda, "all inputs must be CUDA"
        assert u.device == X.device == W_V.device, "u/X/W_V must be on same device"
        assert D_H in (16, 32, 64, 128, 256), f"D_H {D_H} not supported"
        dcode = _lib.dtype_code(u.dtype)
        u, X, W_V = (_aligned(t.contiguous()) for t in (u, X, W_V))
        plan = _absorb_plan(T_q, T_k, H, D_KV, D_H, u.device, cu_seqlens_q, cu_seqlens_k,
                            q_chunk_indices, validate)
        O = torch.empty((T_q, H, D_H), dtype=u.dtype, device=u.device)
        LSE = torch.empty((T_q, H), dtype=torch.float32, device=u.device)
        L = _lib.lib()
        ws = _workspace(L.vafa_absorb_fwd_workspace(plan.info, D_KV, D_H), u.device)
        _lib.check(L.vafa_absorb_fwd(
            u.data_ptr(), X.data_ptr(), W_V.data_ptr(), O.data_ptr(), LSE.data_ptr(),
            plan.items.data_ptr(), plan.info, D_KV, D_H, dcode, float(scale),
            ws.data_ptr() if ws.numel() else None, ws.numel(), _lib.stream_ptr(u.device)))
        ctx.save_for_backward(u, X, W_V, O, LSE)
        ctx.plan = plan
        ctx.scale = scale
        return O

    @staticmethod
    def backward(ctx, dO):
        u, X, W_V, O, LSE = ctx.saved_tensors
        du, dX, dW_V = _absorb_bwd(u, X, W_V, O, LSE, dO, ctx.plan, ctx.scale)
        return du, dX, dW_V, None, None, None, None, None, None


def target_attn_inner(
    u: torch.Tensor,
    X: torch.Tensor,
    W_V: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    scale: Optional[float] = None,
    q_chunk_indices: Optional[torch.Tensor] = None,
    k_chunk_indices: Optional[torch.Tensor] = None,
    validate: bool = True,
) -> torch.Tensor:
    """Inner entry on projected ``u [T_q,H,D_KV]`` (ta/interface.py:324-354)."""
    if scale is None:
        scale = 1.0 / math.sqrt(W_V.shape[2])
    return _TargetAttnFunction.apply(
        u, X, W_V, cu_seqlens_q, cu_seqlens_k, float(scale),
        q_chunk_indices, k_chunk_indices, validate)


def _project_native(q_raw: torch.Tensor, W_Q: torch.Tensor, W_K: torch.Tensor) -> bool:
    """Whether ``vafa_absorb_project_fwd/_bwd`` take these operands: CUDA,
    one 16-bit dtype, D_Q, D_KV and D_H multiples of 8."""
    d_q = q_raw.shape[1]
    d_kv, _, D_H = W_K.shape
    return (q_raw.is_cuda and q_raw.dtype in (torch.bfloat16, torch.float16)
            and W_Q.dtype == q_raw.dtype and W_K.dtype == q_raw.dtype
            and d_q % 8 == 0 and d_kv % 8 == 0 and D_H % 8 == 0)


class _Project(torch.autograd.Function):
    """q_proj = q_raw W_Q, u[t,h,:] = q_proj[t,h,:] W_K[:,h,:]^T
    (ta/interface.py:434-435) for 16-bit operands, forward and backward on
    the row-GEMM and weight-gradient kernels of ``vafa_absorb_project_fwd`` /
    ``vafa_absorb_project_bwd``.  Each product is rounded once to the input
    dtype, as the reference's 16-bit GEMMs and their autograd backward
    (dq_proj = du W_K per head, dq_raw = dq_proj W_Q^T, dW_Q = q_raw^T dq_proj,
    dW_K = du^T q_proj per head); the weight gradients are summed over fixed
    token chunks in order (deterministic)."""

    @staticmethod
    def forward(ctx, q_raw: torch.Tensor, W_Q: torch.Tensor, W_K: torch.Tensor) -> torch.Tensor:
        T_q, d_q = q_raw.shape
        _, H, D_H = W_Q.shape
        d_kv = W_K.shape[0]
        L = _lib.lib()
        q_raw = _aligned(q_raw.contiguous())
        W_Q = _aligned(W_Q.contiguous())
        W_K = _aligned(W_K.contiguous())
        q_proj = torch.empty((T_q, H * D_H), dtype=q_raw.dtype, device=q_raw.device)
        u = torch.empty((T_q, H, d_kv), dtype=q_raw.dtype, device=q_raw.device)
        ws = _workspace(L.vafa_absorb_project_workspace(T_q, H, d_q, d_kv, D_H, 0), q_raw.device)
        _lib.check(L.vafa_absorb_project_fwd(
            q_raw.data_ptr(), W_Q.data_ptr(), W_K.data_ptr(), q_proj.data_ptr(), u.data_ptr(),
            T_q, H, d_q, d_kv, D_H, _lib.dtype_code(q_raw.dtype), ws.data_ptr(), ws.numel(),
            _lib.stream_ptr(q_raw.device)))
        ctx.save_for_backward(q_raw, W_Q, W_K, q_proj)
        return u

    @staticmethod
    def backward(ctx, du: torch.Tensor):
        q_raw, W_Q, W_K, q_proj = ctx.saved_tensors
        T_q, d_q = q_raw.shape
        d_kv, H, D_H = W_K.shape
        need_q, need_wq, need_wk = ctx.needs_input_grad[:3]
        du = _aligned(du.contiguous())
        dq = torch.empty_like(q_raw) if need_q else None
        dwq = torch.empty_like(W_Q) if need_wq else None
        dwk = torch.empty_like(W_K) if need_wk else None
        L = _lib.lib()
        ws = _workspace(L.vafa_absorb_project_workspace(T_q, H, d_q, d_kv, D_H, 1), du.device)

        def ptr(t):
            return t.data_ptr() if t is not None else None

        _lib.check(L.vafa_absorb_project_bwd(
            q_raw.data_ptr(), W_Q.data_ptr(), W_K.data_ptr(), q_proj.data_ptr(), du.data_ptr(),
            ptr(dq), ptr(dwq), ptr(dwk), T_q, H, d_q, d_kv, D_H, _lib.dtype_code(du.dtype),
            ws.data_ptr(), ws.numel(), _lib.stream_ptr(du.device)))
        return dq, dwq, dwk


def _fold_native(q_raw, X, W_Q, W_K, W_V) -> bool:
    """Whether packed_target_attn can run with u folded into the attention
    kernel (vafa_absorb_fwd_fold): the native projection's operands, X and
    W_V of the same dtype on the same device, and a shape of the folded
    matrix-core kernel."""
    if not _project_native(q_raw, W_Q, W_K):
        return False
    if X.dtype != q_raw.dtype or W_V.dtype != q_raw.dtype or not (X.is_cuda and W_V.is_cuda):
        return False
    if not (q_raw.device == X.device == W_Q.device == W_K.device == W_V.device):
        return False
    d_kv, H, D_H = W_K.shape
    return bool(_lib.lib().vafa_absorb_fold_supported(H, d_kv, D_H,
                                                      _lib.dtype_code(q_raw.dtype)))


class _FoldedTargetAttn(torch.autograd.Function):
    """packed_target_attn with the u projection folded into the attention
    forward (ta/interface.py:429-435 followed by ta/interface.py:141-321).

    Forward: q_proj = q_raw W_Q (row-GEMM kernel, rounded to the input dtype),
    then vafa_absorb_fwd_fold, whose workgroups form u = q_proj_h W_K,h^T for
    their own rows on the matrix cores -- u is never written to memory.
    Backward: u is formed once from the saved q_proj (vafa_absorb_project_u,
    the same products), then the inner backward gives du / dX / dW_V and the
    projection backward dq_raw / dW_Q / dW_K, as the unfused path."""

    @staticmethod
    def forward(ctx, q_raw, X, W_Q, W_K, W_V, cu_seqlens_q, cu_seqlens_k, scale,
                q_chunk_indices, k_chunk_indices, validate):
        T_q, d_q = q_raw.shape
        T_k, d_kv = X.shape
        _, H, D_H = W_Q.shape
        dcode = _lib.dtype_code(q_raw.dtype)
        q_raw, X, W_Q, W_K, W_V = (_aligned(t.contiguous()) for t in (q_raw, X, W_Q, W_K, W_V))
        plan = _absorb_plan(T_q, T_k, H, d_kv, D_H, X.device, cu_seqlens_q, cu_seqlens_k,
                            q_chunk_indices, validate)
        L = _lib.lib()
        st = _lib.stream_ptr(X.device)
        q_proj = torch.empty((T_q, H * D_H), dtype=q_raw.dtype, device=q_raw.device)
        pws = _workspace(L.vafa_absorb_project_workspace(T_q, H, d_q, d_kv, D_H, 0), X.device)
        _lib.check(L.vafa_absorb_project_fwd(
            q_raw.data_ptr(), W_Q.data_ptr(), W_K.data_ptr(), q_proj.data_ptr(), None,
            T_q, H, d_q, d_kv, D_H, dcode, pws.data_ptr(), pws.numel(), st))
        O = torch.empty((T_q, H, D_H), dtype=q_raw.dtype, device=X.device)
        LSE = torch.empty((T_q, H), dtype=torch.float32, device=X.device)
        ws = _workspace(L.vafa_absorb_fwd_fold_workspace(plan.info, d_kv, D_H), X.device)
        _lib.check(L.vafa_absorb_fwd_fold(
            q_proj.data_ptr(), W_K.data_ptr(), X.data_ptr(), W_V.data_ptr(), O.data_ptr(),
            LSE.data_ptr(), plan.items.data_ptr(), plan.info, d_kv, D_H, dcode, float(scale),
            ws.data_ptr() if ws.numel() else None, ws.numel(), st))
        ctx.save_for_backward(q_raw, W_Q, W_K, q_proj, X, W_V, O, LSE)
        ctx.plan = plan
        ctx.scale = scale
        return O

    @staticmethod
    def backward(ctx, dO):
        q_raw, W_Q, W_K, q_proj, X, W_V, O, LSE = ctx.saved_tensors
        T_q, d_q = q_raw.shape
        d_kv, H, D_H = W_K.shape
        L = _lib.lib()
        st = _lib.stream_ptr(X.device)
        u = torch.empty((T_q, H, d_kv), dtype=q_raw.dtype, device=X.device)
        _lib.check(L.vafa_absorb_project_u(q_proj.data_ptr(), W_K.data_ptr(), u.data_ptr(), T_q,
                                           H, d_kv, D_H, _lib.dtype_code(u.dtype), st))
        du, dX, dW_V = _absorb_bwd(u, X, W_V, O, LSE, dO, ctx.plan, ctx.scale)
        need_q, _, need_wq, need_wk = ctx.needs_input_grad[:4]
        dq = torch.empty_like(q_raw) if need_q else None
        dwq = torch.empty_like(W_Q) if need_wq else None
        dwk = torch.empty_like(W_K) if need_wk else None
        if need_q or need_wq or need_wk:
            ws = _workspace(L.vafa_absorb_project_workspace(T_q, H, d_q, d_kv, D_H, 1), X.device)
            _lib.check(L.vafa_absorb_project_bwd(
                q_raw.data_ptr(), W_Q.data_ptr(), W_K.data_ptr(), q_proj.data_ptr(),
                du.data_ptr(), _lib.ptr(dq), _lib.ptr(dwq), _lib.ptr(dwk), T_q, H, d_q, d_kv,
                D_H, _lib.dtype_code(du.dtype), ws.data_ptr(), ws.numel(), st))
        return dq, dX, dwq, dwk, dW_V, None, None, None, None, None, None


def _project_u(q_raw: torch.Tensor, W_Q: torch.Tensor, W_K: torch.Tensor) -> torch.Tensor:
    """u[t,h,:] = (q_raw[t] W_Q[:,h,:]) W_K[:,h,:]^T (ta/interface.py:434-435),
    contiguous ``[T_q, H, d_kv]``.

    16-bit operands with D_Q, D_KV, D_H multiples of 8 run on ``_Project``
    (both directions in this library's kernels).  Other operands (fp32, odd
    widths) take the reference's own formulation on torch's GEMMs: q_proj =
    q_raw @ W_Q, then u = q_proj @ blockdiag(W_K[:,h,:]^T), ONE GEMM that
    writes u token-major (for finite q_proj the zero blocks add exact zeros
    to each fp32 sum, so every u element is the same sum of products as per
    head).
    """
    if _project_native(q_raw, W_Q, W_K):
        return _Project.apply(q_raw, W_Q, W_K)
    T_q, d_q = q_raw.shape
    _, H, D_H = W_Q.shape
    q_proj = q_raw @ W_Q.reshape(d_q, H * D_H)
    blocks = torch.block_diag(*[W_K[:, h, :].t() for h in range(H)])
    return (q_proj @ blocks).view(T_q, H, W_K.shape[0])


def packed_target_attn(
    q_raw: torch.Tensor,
    X: torch.Tensor,
    W_Q: torch.Tensor,
    W_K: torch.Tensor,
    W_V: torch.Tensor,
    *,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    cu_seqlens_k: Optional[torch.Tensor] = None,
    q_seqinfo: Optional[torch.Tensor] = None,
    k_seqinfo: Optional[torch.Tensor] = None,
    q_chunk_indices: Optional[torch.Tensor] = None,
    k_chunk_indices: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    bf16: bool = False,
    validate: bool = True,
) -> torch.Tensor:
    """Full ragged target attention with matrix absorption (ta/interface.py:357-445).

    q_raw ``[T_q,d_q]`` or ``[1,T_q,d_q]``; X ``[T_k,d_kv]`` or ``[1,T_k,d_kv]``;
    W_Q ``[d_q,H,D_H]``, W_K/W_V ``[d_kv,H,D_H]``.  Returns O ``[T_q,H,D_H]``
    in the compute dtype (bf16 when ``bf16=True``, else the input dtype).
    """
    if q_raw.dim() == 3:
        assert q_raw.shape[0] == 1, "batch must be 1 for packed varlen"
        q_raw = q_raw.squeeze(0)
    if X.dim() == 3:
        assert X.shape[0] == 1
        X = X.squeeze(0)

    T_q, d_q = q_raw.shape
    T_k, d_kv = X.shape
    d_q_wq, H, D_H = W_Q.shape
    d_kv_wk, H_wk, D_H_wk = W_K.shape
    d_kv_wv, H_wv, D_H_wv = W_V.shape
    assert d_q_wq == d_q, f"W_Q[0]={d_q_wq} != d_q={d_q}"
    assert d_kv_wk == d_kv and d_kv_wv == d_kv, "W_K/W_V d_kv mismatch"
    assert H == H_wk == H_wv, "H mismatch across W_Q/W_K/W_V"
    assert D_H == D_H_wk == D_H_wv, "D_H mismatch across W_Q/W_K/W_V"

    if cu_seqlens_q is None:
        assert q_seqinfo is not None
        cu_seqlens_q = _seqinfo_to_cu(q_seqinfo)
    if cu_seqlens_k is None:
        assert k_seqinfo is not None
        cu_seqlens_k = _seqinfo_to_cu(k_seqinfo)

    if bf16:
        q_raw, X, W_Q, W_K, W_V = (t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)
                                   for t in (q_raw, X, W_Q, W_K, W_V))

    if scale is None:
        scale = 1.0 / math.sqrt(D_H)
    if _fold_native(q_raw, X, W_Q, W_K, W_V):
        return _FoldedTargetAttn.apply(
            q_raw, X, W_Q, W_K, W_V, cu_seqlens_q, cu_seqlens_k, float(scale),
            q_chunk_indices, k_chunk_indices, validate)
    u = _project_u(q_raw, W_Q, W_K)
    return target_attn_inner(
        u, X, W_V, cu_seqlens_q, cu_seqlens_k, scale,
        q_chunk_indices=q_chunk_indices, k_chunk_indices=k_chunk_indices, validate=validate)


def _seqinfo_to_cu(seqinfo: torch.Tensor) -> torch.Tensor:
    """[n_seg] lengths -> [n_seg+1] int32 (ta/interface.py:448-454: asserts only)."""
    assert seqinfo.dim() == 1 and seqinfo.numel() >= 1
    s = _lib.as_host_i64(seqinfo)
    cu = np.zeros(s.size + 1, dtype=np.int64)
    cu[1:] = np.cumsum(s)
    return torch.from_numpy(cu.astype(np.int32)).to(seqinfo.device)
