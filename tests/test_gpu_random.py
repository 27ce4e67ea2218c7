"""Seeded random shapes through both operators against the oracle.

Each case draws segment lengths (empty segments included), head count, head
dim / widths and dtype from a fixed seed, runs forward and backward through
the public entry points (C ABI underneath) and checks every output and
gradient with the parity bounds of tests/parity.py.  The shapes cover the
matrix-core paths' edges: tails of every tile size, split and unsplit key
ranges, head counts that do not divide 64, widths that are padded.

Varlen gradients in 16-bit are held to the reference algorithm's own error
(assert_within_reference_numerics): a segment with a handful of keys against
hundreds of queries gives those keys dK / dV sums of magnitude ~10 (bf16
spacing 0.0625 there) over P and dS that the reference rounds to bf16 before
the products (fa/kernels.py:345, 480, 489), while rms(ref) stays below 1, so
neither the floor-subtracted nor the rms-relative form of the absolute bound
applies to them.
"""
import numpy as np
import pytest
import torch

from parity import assert_close, assert_within_reference_numerics
from test_gpu_absorb import NAMES as ABSORB_NAMES
from test_gpu_absorb import run_case as absorb_case
from test_gpu_varlen import run_case as varlen_case

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _varlen_draw(seed):
    r = np.random.default_rng(1000 + seed)
    n = int(r.integers(1, 6))
    q = [int(x) for x in r.integers(0, 300, size=n)]
    k = [int(x) for x in r.integers(0, 700, size=n)]
    if r.random() < 0.3:  # a long key range: split-K partials
        k[int(r.integers(0, n))] = int(r.integers(4097, 12000))
    H = int(r.choice([1, 2, 3, 4, 6]))
    D = int(r.choice([16, 32, 64, 128, 256]))
    dt = DTYPES[int(r.integers(0, 3))]
    return q, k, H, D, dt


@pytest.mark.parametrize("seed", range(24))
def test_varlen_random_shapes(device, seed):
    q, k, H, D, dt = _varlen_draw(seed)
    print(f"[varlen random {seed}] q={q} k={k} H={H} D={D} {dt}", flush=True)
    if dt == torch.float32:
        got, ref = varlen_case(q, k, H, D, dt, device, seed=seed)
        for n, a, r in zip(("o", "dq", "dk", "dv"), got, ref):
            assert_close(n, a, r)
        return
    got, ref, emul = varlen_case(q, k, H, D, dt, device, seed=seed, reference_numerics=True)
    assert_close("o", got[0], ref[0])
    for n, a, r, em in zip(("dq", "dk", "dv"), got[1:], ref[1:], emul):
        assert_within_reference_numerics(n, a, r, em)


def _absorb_draw(seed):
    r = np.random.default_rng(2000 + seed)
    n = int(r.integers(1, 6))
    q = [int(x) for x in r.integers(0, 24, size=n)]
    k = [int(x) for x in r.integers(1, 900, size=n)]  # q > 0 needs k > 0
    H = int(r.choice([1, 2, 3, 5, 8, 12, 16, 24]))
    D_H = int(r.choice([16, 32, 64, 128]))
    d_kv = int(r.integers(4, 513))
    dt = DTYPES[int(r.integers(0, 3))]
    return q, k, H, D_H, d_kv, dt


@pytest.mark.parametrize("seed", range(24))
def test_absorb_random_shapes(device, seed):
    q, k, H, D_H, d_kv, dt = _absorb_draw(seed)
    print(f"[absorb random {seed}] q={q} k={k} H={H} D_H={D_H} d_kv={d_kv} {dt}", flush=True)
    got, ref = absorb_case(q, k, dt, device, d_q=64, d_kv=d_kv, H=H, D_H=D_H, seed=seed)
    for n, a, r in zip(ABSORB_NAMES, got, ref):
        assert_close(n, a, r)
