"""Packed variable-length FlashAttention -- drop-in for
``triton_fa_varlen_v2.packed_varlen_attn`` (fa/interface.py:344-392).

Same signature, same input normalisation (fa/interface.py:121-150), same
cu_seqlens / seqinfo rules and error types (fa/interface.py:74-118,
158-175).  Compute runs in ``libvafa.so`` (hand-written gfx950 kernels): a
host plan built from cu_seqlens drives a forward kernel over query tiles with
split-K partials plus an LSE combine, and a deterministic backward (row-dot
delta, dQ over query tiles with ordered split sums, dK/dV over key tiles).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib

_VALIDATE_CU_SEQLENS = True


def set_validate_cu_seqlens(enabled: bool) -> None:
    """Toggle the host-side cu_seqlens validation (fa/interface.py:68-71)."""
    global _VALIDATE_CU_SEQLENS
    _VALIDATE_CU_SEQLENS = bool(enabled)


def _seqinfo_to_cu_seqlens(seqinfo: torch.Tensor) -> torch.Tensor:
    """[n_seg] lengths -> [n_seg+1] int32 cu_seqlens (fa/interface.py:74-93)."""
    if seqinfo.dim() != 1:
        raise ValueError(f"seqinfo must be 1-D [n_seg], got shape {tuple(seqinfo.shape)}")
    cu = _lib.seqinfo_to_cu(_lib.as_host_i64(seqinfo))
    return torch.from_numpy(cu).to(seqinfo.device)


def _validate_cu_seqlens(cu_host, shape, T: int, name: str) -> None:
    """fa/interface.py:96-118, on the host copy taken once per call."""
    if not _VALIDATE_CU_SEQLENS:
        return
    if len(shape) != 1:
        raise ValueError(f"{name}: must be 1-D, got shape {tuple(shape)}")
    _lib.validate_cu(cu_host, T, name)


def _normalize_qkv(x: torch.Tensor, name: str) -> Tuple[torch.Tensor, bool]:
    """[1,T,H,D] or [T,H,D] -> contiguous [T,H,D] (fa/interface.py:121-150)."""
    if x.dim() == 4:
        if x.shape[0] != 1:
            raise ValueError(
                f"{name}: 4-D input must have batch=1 (packed varlen), "
                f"got shape {tuple(x.shape)}")
        x = x.squeeze(0)
        was_4d = True
    elif x.dim() == 3:
        was_4d = False
    else:
        raise ValueError(f"{name}: expected 3-D [T,H,D] or 4-D [1,T,H,D], got {x.dim()}-D")
    T, H, D = x.shape
    if x.stride(-1) != 1 or x.stride(1) != D or x.stride(0) != H * D:
        x = x.contiguous()
    return x, was_4d


def _aligned(x: torch.Tensor) -> torch.Tensor:
    """The kernels issue 16-byte vector loads: realign odd views."""
    if x.data_ptr() % 16 != 0:
        x = x.clone()
    return x


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 0), dtype=torch.uint8, device=device)


def _check_tokens(info, T_q: int, T_k: int) -> None:
    # Bounds guard that stays on even when validation is disabled: a plan
    # reaching past the tensors would read out of bounds on the GPU.
    if info.T_q > T_q or info.T_k > T_k:
        raise ValueError(
            f"cu_seqlens address {info.T_q} query / {info.T_k} key tokens but the inputs "
            f"hold {T_q} / {T_k}")


class _PackedVarlenAttnFunction(torch.autograd.Function):
    """Autograd wrapper (fa/interface.py:153-341)."""

    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens_q, cu_seqlens_k, scale):
        T_q, H, D = q.shape
        T_k = k.shape[0]
        assert k.shape == (T_k, H, D), f"K shape mismatch: {k.shape} vs expected ({T_k},{H},{D})"
        assert v.shape == (T_k, H, D), f"V shape mismatch: {v.shape} vs expected ({T_k},{H},{D})"
        assert q.dtype == k.dtype == v.dtype, "q/k/v must share dtype"
        assert q.dtype.is_floating_point, f"q/k/v must be float, got {q.dtype}"
        assert q.is_cuda, "packed_varlen_attn requires GPU tensors"
        assert k.device == q.device and v.device == q.device, "q/k/v must be on the same device"
        assert D in (16, 32, 64, 128, 256), f"head_dim {D} not supported (try 64/128/256)"
        dcode = _lib.dtype_code(q.dtype)

        n_seg = cu_seqlens_q.numel() - 1
        assert cu_seqlens_k.numel() - 1 == n_seg, \
            f"segment count mismatch: q has {n_seg}, k has {cu_seqlens_k.numel()-1}"
        # work that does not need the host copy of cu_seqlens goes first: the
        # copy waits for the GPU work already queued, and what follows it runs
        # while the GPU is idle
        q, k, v = _aligned(q), _aligned(k), _aligned(v)
        o = torch.empty_like(q)
        lse = torch.empty((T_q, H), dtype=torch.float32, device=q.device)
        L = _lib.lib()
        cu_q_h, cu_k_h = _lib.as_host_i64_pair(cu_seqlens_q, cu_seqlens_k)
        _validate_cu_seqlens(cu_q_h, cu_seqlens_q.shape, T_q, "cu_seqlens_q")
        _validate_cu_seqlens(cu_k_h, cu_seqlens_k.shape, T_k, "cu_seqlens_k")
        if cu_q_h.ndim != 1 or cu_q_h.size < 2:
            raise ValueError("cu_seqlens_q: must be 1-D with at least 2 elements")

        plan = _lib.device_plan("varlen", cu_q_h, cu_k_h, (H, D), q.device)
        _check_tokens(plan.info, T_q, T_k)
        ws = _workspace(L.vafa_varlen_fwd_workspace(plan.info, D), q.device)
        _lib.check(L.vafa_varlen_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            plan.items.data_ptr(), plan.info, D, dcode, float(scale),
            ws.data_ptr() if ws.numel() else None, ws.numel(), _lib.stream_ptr(q.device)))
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.plan = plan
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        plan = ctx.plan
        T_q, H, D = q.shape
        if do.stride(-1) != 1 or not do.is_contiguous():
            do = do.contiguous()
        if do.dtype != q.dtype:
            do = do.to(q.dtype)
        do = _aligned(do)
        dq = torch.empty_like(q)
        dk = torch.empty_like(k)
        dv = torch.empty_like(v)
        L = _lib.lib()
        ws = _workspace(L.vafa_varlen_bwd_workspace(plan.info, D), q.device)
        _lib.check(L.vafa_varlen_bwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
            lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
            plan.items.data_ptr(), plan.info, D, _lib.dtype_code(q.dtype), float(ctx.scale),
            ws.data_ptr() if ws.numel() else None, ws.numel(), _lib.stream_ptr(q.device)))
        return dq, dk, dv, None, None, None


def packed_varlen_attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    cu_seqlens_k: Optional[torch.Tensor] = None,
    q_seqinfo: Optional[torch.Tensor] = None,
    k_seqinfo: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Packed-varlen attention with block-diagonal (per-segment) masking.

    Args mirror fa/interface.py:344-392: q ``[1,T_q,H,D]`` or ``[T_q,H,D]``,
    k/v likewise; ``cu_seqlens_*`` (preferred) or ``*_seqinfo``; scale
    defaults to ``1/sqrt(D)``.  Output follows q's rank.
    """
    q3, q_was_4d = _normalize_qkv(q, "q")
    k3, _ = _normalize_qkv(k, "k")
    v3, _ = _normalize_qkv(v, "v")

    if cu_seqlens_q is None:
        if q_seqinfo is None:
            raise ValueError("must provide either cu_seqlens_q or q_seqinfo")
        cu_seqlens_q = _seqinfo_to_cu_seqlens(q_seqinfo)
    if cu_seqlens_k is None:
        if k_seqinfo is None:
            raise ValueError("must provide either cu_seqlens_k or k_seqinfo")
        cu_seqlens_k = _seqinfo_to_cu_seqlens(k_seqinfo)

    if scale is None:
        scale = 1.0 / math.sqrt(q3.shape[-1])

    o3 = _PackedVarlenAttnFunction.apply(q3, k3, v3, cu_seqlens_q, cu_seqlens_k, float(scale))
    return o3.unsqueeze(0) if q_was_4d else o3


class BackwardStages:
    """The three backward stages of packed_varlen_attn as separate launches.

    For profiling and for callers that schedule the backward themselves (the
    dQ and dK/dV stages are independent once delta is written).  Built from
    forward inputs; ``run(stage)`` launches one stage on the current stream:
    0 = delta, 1 = dQ (+ split sums), 2 = dK/dV.
    """

    def __init__(self, q, k, v, do, cu_seqlens_q, cu_seqlens_k, scale=None):
        q3, _ = _normalize_qkv(q, "q")
        k3, _ = _normalize_qkv(k, "k")
        v3, _ = _normalize_qkv(v, "v")
        self.D = q3.shape[-1]
        self.scale = float(scale if scale is not None else 1.0 / math.sqrt(self.D))
        cu_q_h = _lib.as_host_i64(cu_seqlens_q)
        cu_k_h = _lib.as_host_i64(cu_seqlens_k)
        _lib.validate_cu(cu_q_h, q3.shape[0], "cu_seqlens_q")
        _lib.validate_cu(cu_k_h, k3.shape[0], "cu_seqlens_k")
        H = q3.shape[1]
        self.plan = _lib.device_plan("varlen", cu_q_h, cu_k_h, (H, self.D), q3.device)
        self.q, self.k, self.v = _aligned(q3), _aligned(k3), _aligned(v3)
        self.do = _aligned(do.reshape(q3.shape).contiguous().to(q3.dtype))
        # forward through the C ABI (O and the log2-domain LSE)
        self.lse = torch.empty((q3.shape[0], H), dtype=torch.float32, device=q3.device)
        L = _lib.lib()
        fws = _workspace(L.vafa_varlen_fwd_workspace(self.plan.info, self.D), q3.device)
        o2 = torch.empty_like(self.q)
        _lib.check(L.vafa_varlen_fwd(
            self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), o2.data_ptr(),
            self.lse.data_ptr(), self.plan.items.data_ptr(), self.plan.info, self.D,
            _lib.dtype_code(q3.dtype), self.scale, fws.data_ptr() if fws.numel() else None,
            fws.numel(), _lib.stream_ptr(q3.device)))
        self.o = o2
        self.dq = torch.empty_like(self.q)
        self.dk = torch.empty_like(self.k)
        self.dv = torch.empty_like(self.v)
        self.ws = _workspace(L.vafa_varlen_bwd_workspace(self.plan.info, self.D), q3.device)

    def run(self, stage: int) -> None:
        L = _lib.lib()
        _lib.check(L.vafa_varlen_bwd_stage(
            int(stage), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
            self.o.data_ptr(), self.do.data_ptr(), self.lse.data_ptr(), self.dq.data_ptr(),
            self.dk.data_ptr(), self.dv.data_ptr(), self.plan.items.data_ptr(), self.plan.info,
            self.D, _lib.dtype_code(self.q.dtype), self.scale,
            self.ws.data_ptr() if self.ws.numel() else None, self.ws.numel(),
            _lib.stream_ptr(self.q.device)))
