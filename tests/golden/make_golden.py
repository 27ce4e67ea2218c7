"""Writes config1_oracle_summary.json: a regression pin of the CPU oracle on
configs[0] (packed varlen self-attention, fp32, lens {17,64,128,200}, H=4,
D=64, scale 1/8, q/k/v/dO ~ N(0,1) from numpy default_rng(2024)).

The summary holds, per output (o, lse, dq, dk, dv, computed in float64),
the sum, the absolute sum and 64 samples at fixed flat indices.
Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

LENS = [17, 64, 128, 200]
H, D, SEED = 4, 64, 2024


def config1_inputs():
    rng = np.random.default_rng(SEED)
    T = sum(LENS)
    q, k, v, do = (rng.standard_normal((T, H, D)) for _ in range(4))
    cu = np.zeros(len(LENS) + 1, dtype=np.int64)
    cu[1:] = np.cumsum(LENS)
    return q, k, v, do, cu


def config1_outputs():
    from oracle import varlen as ov
    q, k, v, do, cu = config1_inputs()
    sc = 1.0 / math.sqrt(D)
    o, lse = ov.forward(q, k, v, cu, cu, sc, np.float64)
    dq, dk, dv = ov.backward(q, k, v, do, cu, cu, sc, np.float64)
    return {"o": o, "lse": lse, "dq": dq, "dk": dk, "dv": dv}


def summarize(a):
    flat = np.asarray(a, dtype=np.float64).ravel()
    idx = np.linspace(0, flat.size - 1, 64).astype(np.int64)
    return {"sum": float(flat.sum()), "abs_sum": float(np.abs(flat).sum()),
            "samples": flat[idx].tolist()}


if __name__ == "__main__":
    out = {name: summarize(a) for name, a in config1_outputs().items()}
    with open(os.path.join(HERE, "config1_oracle_summary.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote config1_oracle_summary.json")
