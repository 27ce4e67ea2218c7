"""Seeded synthetic workloads for the five benchmark configurations.

Lengths come from ``numpy.random.default_rng(seed)``; values are N(0,1) from a
``torch.Generator`` seeded the same way on the target device (large configs
never materialise on the host).  Weights of the absorb configs are
Xavier-uniform ``[256, 256]`` viewed as ``[256, H, D_H]``.
"""
from __future__ import annotations

import dataclasses
import math
from typing import List, Optional

import numpy as np
import torch


@dataclasses.dataclass
class VarlenCase:
    name: str
    q_lens: List[int]
    k_lens: List[int]
    H: int
    D: int
    dtype: torch.dtype
    seed: int = 0

    @property
    def flops_fwd(self) -> float:
        """4 H D sum(Lq Lk) (fa-tools/benchmark_packed_varlen_flash_attn.py:289-292)."""
        return 4.0 * self.H * self.D * float(np.dot(self.q_lens, self.k_lens))

    @property
    def flops_bwd(self) -> float:
        """10 H D sum(Lq Lk): five GEMMs of the backward."""
        return 2.5 * self.flops_fwd

    def bytes_fwd(self) -> float:
        """Algorithmic HBM bytes: read q, k, v once, write o (2 B elements)."""
        es = torch.tensor([], dtype=self.dtype).element_size()
        return float(self.H * self.D * es * 2 * (sum(self.q_lens) + sum(self.k_lens)))


@dataclasses.dataclass
class AbsorbCase:
    name: str
    q_lens: List[int]
    k_lens: List[int]
    H: int
    D_H: int
    D_in: int
    dtype: torch.dtype
    seed: int = 0

    def bytes_fwd(self) -> float:
        """Inner-op bytes |X| + |u| + |W_V| + |O| + |LSE| with X read once."""
        es = torch.tensor([], dtype=self.dtype).element_size()
        Tq, Tk = sum(self.q_lens), sum(self.k_lens)
        return float(es * (Tk * self.D_in + Tq * self.H * self.D_in
                           + self.D_in * self.H * self.D_H + Tq * self.H * self.D_H)
                     + 4 * Tq * self.H)

    @property
    def flops_fwd(self) -> float:
        lq = np.asarray(self.q_lens, dtype=np.float64)
        lk = np.asarray(self.k_lens, dtype=np.float64)
        return self.H * (4.0 * self.D_in * float(np.dot(lq, lk))
                         + 2.0 * self.D_in * self.D_H * float(lq.sum()))


def _log_uniform_int(rng, lo, hi, n):
    x = np.exp(rng.uniform(math.log(lo), math.log(hi), size=n))
    return np.clip(np.rint(x), lo, hi).astype(np.int64)


def config1(seed: int = 0) -> VarlenCase:
    """CPU plumbing: lens {17,64,128,200}, H=4, D=64, fp32."""
    return VarlenCase("c1_cpu_plumbing", [17, 64, 128, 200], [17, 64, 128, 200], 4, 64,
                      torch.float32, seed)


def config2(seed: int = 0, n_seq: int = 64) -> VarlenCase:
    """Varlen fwd+bwd: 64 seqs, lengths log-uniform in [1, 4096], H=16, D=128, bf16."""
    rng = np.random.default_rng(seed)
    lens = _log_uniform_int(rng, 1, 4096, n_seq).tolist()
    return VarlenCase("c2_varlen_fwd_bwd", lens, lens, 16, 128, torch.bfloat16, seed)


def config2_tokens(seed: int = 0, total: int = 128 * 1024) -> VarlenCase:
    """configs[1] read by its token count ("about 128k total tokens"): the same
    seeded log-uniform draw as config2 (whose 64 sequences are its prefix),
    extended until the packed length reaches ``total`` tokens."""
    rng = np.random.default_rng(seed)
    lens = _log_uniform_int(rng, 1, 4096, 4096)
    n = int(np.searchsorted(np.cumsum(lens), total)) + 1
    lens = lens[:n].tolist()
    return VarlenCase("c2_varlen_fwd_bwd_128k_tokens", lens, lens, 16, 128, torch.bfloat16, seed)


def config3(seed: int = 0, n_seq: int = 256) -> VarlenCase:
    """Split-K forward: Lq ~ U{1..16}, Lk log-uniform in [1024, 32768], H=32, D=128."""
    rng = np.random.default_rng(seed)
    lq = rng.integers(1, 17, size=n_seq).tolist()
    lk = _log_uniform_int(rng, 1024, 32768, n_seq).tolist()
    return VarlenCase("c3_varlen_splitk_fwd", lq, lk, 32, 128, torch.bfloat16, seed)


def config4(seed: int = 0, n: int = 2048) -> AbsorbCase:
    """Absorb: Lq ~ U{1..8}, Lk = clip(round(LogNormal(ln 200, 1)), 1, 2000)."""
    rng = np.random.default_rng(seed)
    lq = rng.integers(1, 9, size=n).tolist()
    lk = np.clip(np.rint(rng.lognormal(math.log(200.0), 1.0, size=n)), 1, 2000)
    return AbsorbCase("c4_absorb", lq, lk.astype(np.int64).tolist(), 8, 32, 256,
                      torch.bfloat16, seed)


def config5(seed: int = 0, n: int = 8192) -> AbsorbCase:
    """Absorb skewed: Lq ~ U{1..32}, Lk = clip(Zipf(1.2), 1, 8192), forward only."""
    rng = np.random.default_rng(seed)
    lq = rng.integers(1, 33, size=n).tolist()
    lk = np.clip(rng.zipf(1.2, size=n), 1, 8192).astype(np.int64).tolist()
    return AbsorbCase("c5_absorb_skewed", lq, lk, 8, 32, 256, torch.bfloat16, seed)


def cu_from_lens(lens, device=None) -> torch.Tensor:
    cu = np.zeros(len(lens) + 1, dtype=np.int64)
    cu[1:] = np.cumsum(lens)
    return torch.from_numpy(cu.astype(np.int32)).to(device or "cpu")


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def varlen_tensors(case: VarlenCase, device, with_grad_out: bool = False,
                   dtype: Optional[torch.dtype] = None):
    """q, k, v (and dO) ~ N(0,1) in ``dtype`` (default the case dtype) on ``device``."""
    dt = dtype or case.dtype
    g = _gen(device, case.seed)
    Tq, Tk = sum(case.q_lens), sum(case.k_lens)
    mk = lambda T: torch.randn(T, case.H, case.D, generator=g, device=device,
                               dtype=torch.float32).to(dt)
    q, k, v = mk(Tq), mk(Tk), mk(Tk)
    out = [q, k, v]
    if with_grad_out:
        out.append(mk(Tq))
    return out


def absorb_tensors(case: AbsorbCase, device, d_q: Optional[int] = None,
                   dtype: Optional[torch.dtype] = None):
    """q_raw, X ~ N(0,1); W_Q, W_K, W_V Xavier-uniform [d, H*D_H] viewed [d, H, D_H]."""
    dt = dtype or case.dtype
    g = _gen(device, case.seed)
    Tq, Tk = sum(case.q_lens), sum(case.k_lens)
    d_q = d_q or case.D_in
    f32 = dict(generator=g, device=device, dtype=torch.float32)
    q_raw = torch.randn(Tq, d_q, **f32).to(dt)
    X = torch.randn(Tk, case.D_in, **f32).to(dt)

    def xavier(fan_in):
        bound = math.sqrt(6.0 / (fan_in + case.H * case.D_H))
        w = (torch.rand(fan_in, case.H * case.D_H, **f32) * 2 - 1) * bound
        return w.view(fan_in, case.H, case.D_H).to(dt)

    return q_raw, X, xavier(d_q), xavier(case.D_in), xavier(case.D_in)
