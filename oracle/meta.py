"""Host metadata rules of the reference, restated in numpy (test oracle only).

Integer work: every function here must match the product planner bit-exactly.
"""
from __future__ import annotations

import numpy as np

INT32_MAX = 2_147_483_647


def seqinfo_to_cu(seqinfo) -> np.ndarray:
    """Per-segment lengths -> int32 prefix sums ``[n+1]``.

    Follows fa/interface.py:74-93: 1-D required, non-empty, no negatives,
    int64 cumsum, total must fit int32; raises ValueError otherwise.
    """
    s = np.asarray(seqinfo)
    if s.ndim != 1:
        raise ValueError(f"seqinfo must be 1-D [n_seg], got shape {tuple(s.shape)}")
    if s.size == 0:
        raise ValueError("seqinfo is empty (n_seg=0)")
    s = s.astype(np.int64)
    if (s < 0).any():
        raise ValueError("seqinfo contains negative values")
    cu = np.zeros(s.size + 1, dtype=np.int64)
    cu[1:] = np.cumsum(s)
    if cu[-1] > INT32_MAX:
        raise ValueError(f"total tokens {int(cu[-1])} exceeds int32 range")
    return cu.astype(np.int32)


def validate_cu_seqlens(cu, T: int, name: str) -> None:
    """fa/interface.py:96-118: 1-D, >=2 entries, cu[0]==0, cu[-1]==T, non-decreasing."""
    c = np.asarray(cu)
    if c.ndim != 1:
        raise ValueError(f"{name}: must be 1-D, got shape {tuple(c.shape)}")
    if c.size < 2:
        raise ValueError(f"{name}: must have at least 2 elements (n_seg+1 with n_seg>=1)")
    c = c.astype(np.int64)
    if c[0] != 0:
        raise ValueError(f"{name}[0] must be 0, got {int(c[0])}")
    if c[-1] != T:
        raise ValueError(f"{name}[-1] must equal total tokens {T}, got {int(c[-1])}")
    if (np.diff(c) < 0).any():
        raise ValueError(f"{name} must be non-decreasing (found negative segment length)")


def validate_cu_seqlens_absorb(cu, T: int, name: str) -> None:
    """ta/interface.py:92-106: the same checks as the varlen rule, with the
    absorb operator's texts (1-D with len>=2, [0]==0, [-1]==T, non-decreasing)."""
    c = np.asarray(cu)
    if c.ndim != 1 or c.size < 2:
        raise ValueError(f"{name}: must be 1-D with len>=2, got {tuple(c.shape)}")
    c = c.astype(np.int64)
    if c[0] != 0:
        raise ValueError(f"{name}[0] must be 0")
    if c[-1] != T:
        raise ValueError(f"{name}[-1] must equal total tokens {T}, got {int(c[-1])}")
    if (np.diff(c) < 0).any():
        raise ValueError(f"{name} must be non-decreasing")


def active_segments_have_keys(cu_q, cu_k) -> None:
    """ta/interface.py:109-116: q_len>0 requires k_len>0."""
    lq = np.diff(np.asarray(cu_q, dtype=np.int64))
    lk = np.diff(np.asarray(cu_k, dtype=np.int64))
    if ((lq > 0) & (lk <= 0)).any():
        raise ValueError("segments with q_len > 0 must have k_len > 0")


def chunk_indices(cu, BT: int) -> np.ndarray:
    """Rows ``(seg, block)`` for ``block < ceil(L_seg/BT)``, segment order.

    fa/chunk_indices.py:25-65 and ta/chunk_indices.py:19-54.
    """
    c = np.asarray(cu, dtype=np.int64)
    lens = np.diff(c)
    nb = (lens + BT - 1) // BT
    seg = np.repeat(np.arange(lens.size, dtype=np.int32), nb)
    starts = np.repeat(np.cumsum(nb) - nb, nb)
    blk = (np.arange(int(nb.sum()), dtype=np.int64) - starts).astype(np.int32)
    return np.stack([seg, blk], axis=1).astype(np.int32).reshape(-1, 2)


def split_plan(cu_q, cu_k, BT: int, split_k_block: int, split_threshold: int):
    """Reference long/short split dispatch (fa/chunk_indices.py:172-287).

    Returns ``(short [N,2], split [N,3], combine [N,4])`` with the reference
    row semantics: short rows ``(seg, qblk)`` for segments with
    ``Lk <= threshold``; split rows ``(seg, qblk, ks)`` q-block-major,
    split-minor, one per ``split_k_block`` slice; combine rows
    ``(seg, qblk, first_partial_row, nsplit)``.
    """
    cq = np.asarray(cu_q, dtype=np.int64)
    ck = np.asarray(cu_k, dtype=np.int64)
    lq, lk = np.diff(cq), np.diff(ck)
    short, split, comb = [], [], []
    running = 0
    for s in range(lq.size):
        nb = (int(lq[s]) + BT - 1) // BT
        if lk[s] <= split_threshold:
            short += [(s, t) for t in range(nb)]
            continue
        ns = (int(lk[s]) + split_k_block - 1) // split_k_block
        for t in range(nb):
            split += [(s, t, ks) for ks in range(ns)]
            comb.append((s, t, running + t * ns, ns))
        running += nb * ns
    return (np.array(short, dtype=np.int32).reshape(-1, 2),
            np.array(split, dtype=np.int32).reshape(-1, 3),
            np.array(comb, dtype=np.int32).reshape(-1, 4))
