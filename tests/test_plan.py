"""Host metadata and work plans (CPU): bit-exact against the oracle, plus
coverage invariants checked by brute force."""
import json
import os

import numpy as np
import pytest

from conftest import ROOT
from oracle import meta
from varlenabsorbflashattn_amd import _lib

GOLD = os.path.join(ROOT, "tests", "golden")


def _cu(lens):
    c = np.zeros(len(lens) + 1, dtype=np.int64)
    c[1:] = np.cumsum(lens)
    return c


def _stage1_cases():
    with open(os.path.join(GOLD, "stage1_shapes_subset.jsonl")) as f:
        return [json.loads(l) for l in f if l.strip()]


# ---- oracle pins -------------------------------------------------------------

def test_oracle_chunk_indices_brute_force():
    rng = np.random.default_rng(1)
    for _ in range(50):
        lens = rng.integers(0, 300, size=rng.integers(1, 12))
        bt = int(rng.choice([1, 16, 64, 128]))
        want = [(s, b) for s, L in enumerate(lens) for b in range(-(-int(L) // bt))]
        got = meta.chunk_indices(_cu(lens), bt)
        assert got.tolist() == [list(x) for x in want]


def test_oracle_seqinfo_matches_cumsum_and_errors():
    assert meta.seqinfo_to_cu([3, 0, 5]).tolist() == [0, 3, 3, 8]
    with pytest.raises(ValueError):
        meta.seqinfo_to_cu([])
    with pytest.raises(ValueError):
        meta.seqinfo_to_cu([1, -1])
    with pytest.raises(ValueError):
        meta.seqinfo_to_cu([[1, 2]])
    with pytest.raises(ValueError):
        meta.seqinfo_to_cu([2**31 - 1, 1])


def test_oracle_split_plan_reference_example():
    # Lk = 9000 > 4096 -> 3 slices of 4096; q block of 128 rows: 2 blocks for Lq=200
    short, split, comb = meta.split_plan(_cu([10, 200]), _cu([50, 9000]), 128, 4096, 4096)
    assert short.tolist() == [[0, 0]]
    assert split.tolist() == [[1, 0, 0], [1, 0, 1], [1, 0, 2], [1, 1, 0], [1, 1, 1], [1, 1, 2]]
    assert comb.tolist() == [[1, 0, 0, 3], [1, 1, 3, 3]]


# ---- product vs oracle (bit-exact) --------------------------------------------

@pytest.mark.parametrize("seed", range(8))
def test_seqinfo_to_cu_bit_exact(seed):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, 5000, size=rng.integers(1, 200))
    assert np.array_equal(_lib.seqinfo_to_cu(lens), meta.seqinfo_to_cu(lens))


@pytest.mark.parametrize("bad", [[], [1, -2, 3], [2**31 - 1, 5]])
def test_seqinfo_to_cu_errors_match(bad):
    with pytest.raises(ValueError) as e_ref:
        meta.seqinfo_to_cu(bad)
    with pytest.raises(ValueError) as e_new:
        _lib.seqinfo_to_cu(np.asarray(bad, dtype=np.int64))
    assert str(e_ref.value).split()[0] == str(e_new.value).split()[0]


# (cu, T, expected varlen text, expected absorb text); None = valid.  The texts
# are the reference's: fa/interface.py:108-118 and ta/interface.py:98-106.
VALIDATE_CASES = [
    ([0, 3, 5], 5, None, None),
    ([0, 3, 3, 5], 5, None, None),
    ([1, 3, 5], 5, "cu_seqlens_q[0] must be 0, got 1", "cu_seqlens_q[0] must be 0"),
    ([0, 3, 4], 5, "cu_seqlens_q[-1] must equal total tokens 5, got 4",
     "cu_seqlens_q[-1] must equal total tokens 5, got 4"),
    ([0, 4, 3, 5], 5, "cu_seqlens_q must be non-decreasing (found negative segment length)",
     "cu_seqlens_q must be non-decreasing"),
    ([0], 0, "cu_seqlens_q: must have at least 2 elements (n_seg+1 with n_seg>=1)",
     "cu_seqlens_q: must be 1-D with len>=2, got (1,)"),
    # the first failing rule wins: [0] before [-1] before monotonicity
    ([2, 1, 9], 5, "cu_seqlens_q[0] must be 0, got 2", "cu_seqlens_q[0] must be 0"),
    ([0, 7, 3], 5, "cu_seqlens_q[-1] must equal total tokens 5, got 3",
     "cu_seqlens_q[-1] must equal total tokens 5, got 3"),
]


def _outcome(fn, cu, T):
    try:
        fn(np.array(cu), T, "cu_seqlens_q")
    except ValueError as e:
        return str(e)
    return None


@pytest.mark.parametrize("cu,T,fa_text,ta_text", VALIDATE_CASES)
def test_validate_cu_varlen_texts(cu, T, fa_text, ta_text):
    """Oracle and product both give the varlen operator's exact outcome."""
    assert _outcome(meta.validate_cu_seqlens, cu, T) == fa_text
    assert _outcome(_lib.validate_cu, cu, T) == fa_text


@pytest.mark.parametrize("cu,T,fa_text,ta_text", VALIDATE_CASES)
def test_validate_cu_absorb_texts(cu, T, fa_text, ta_text):
    """Oracle and product both give the absorb operator's exact outcome."""
    assert _outcome(meta.validate_cu_seqlens_absorb, cu, T) == ta_text
    assert _outcome(_lib.validate_cu_absorb, cu, T) == ta_text


ACTIVE_TEXT = "segments with q_len > 0 must have k_len > 0"  # ta/interface.py:116

ACTIVE_CASES = [
    # (cu_q, cu_k, raises): literal cases of ta/interface.py:109-116
    ([0, 2, 2], [0, 5, 5], False),     # a trailing segment with no queries and no keys
    ([0, 2, 3], [0, 5, 5], True),      # 1 query against 0 keys
    ([0, 0, 3], [0, 0, 4], False),     # empty first segment on both sides
    ([0, 0], [0, 7], False),           # keys without queries
    ([0, 4], [0, 0], True),            # the only segment has queries and no keys
    ([0], [0], False),                 # no segments at all
    ([0, 1, 1, 2], [0, 3, 3, 3], True),  # the last segment alone violates it
]


def _active_outcome(fn, cq, ck):
    try:
        fn(np.array(cq), np.array(ck))
        return None
    except ValueError as e:
        return str(e)


@pytest.mark.parametrize("cq,ck,raises", ACTIVE_CASES)
def test_active_segments_have_keys(cq, ck, raises):
    """Oracle (oracle/meta.py) and product (vafa_check_active_have_keys) give
    the reference's outcome and exact text on literal cases."""
    want = ACTIVE_TEXT if raises else None
    assert _active_outcome(meta.active_segments_have_keys, cq, ck) == want
    assert _active_outcome(_lib.check_active_have_keys, cq, ck) == want


def test_active_segments_have_keys_brute_force():
    """Random segment tables with zero lengths on either side: the oracle and
    the product agree with a per-segment loop over the rule."""
    rng = np.random.default_rng(7)
    for _ in range(200):
        n = int(rng.integers(1, 12))
        lq = rng.integers(0, 3, size=n) * rng.integers(0, 2, size=n)
        lk = rng.integers(0, 3, size=n) * rng.integers(0, 2, size=n)
        bad = any(a > 0 and b == 0 for a, b in zip(lq.tolist(), lk.tolist()))
        want = ACTIVE_TEXT if bad else None
        assert _active_outcome(meta.active_segments_have_keys, _cu(lq), _cu(lk)) == want
        assert _active_outcome(_lib.check_active_have_keys, _cu(lq), _cu(lk)) == want


@pytest.mark.parametrize("bt", [16, 64, 128])
def test_chunk_indices_bit_exact(bt):
    rng = np.random.default_rng(bt)
    for _ in range(20):
        lens = rng.integers(0, 700, size=rng.integers(1, 40))
        assert np.array_equal(_lib.chunk_indices(_cu(lens), bt), meta.chunk_indices(_cu(lens), bt))


def test_chunk_indices_real_shapes():
    rec = json.load(open(os.path.join(GOLD, "ta_real_shape_subset.json")))["records"][0]
    for lens, bt in ((rec["q_lens"], 16), (rec["k_lens"], 64)):
        assert np.array_equal(_lib.chunk_indices(_cu(lens), bt), meta.chunk_indices(_cu(lens), bt))


# ---- plan invariants ------------------------------------------------------------

def check_varlen_plan(q_lens, k_lens, H=4, D=64):
    cq, ck = _cu(q_lens), _cu(k_lens)
    p = _lib.plan_varlen(cq, ck, H, D)
    fwd, comb, kv = p.section("fwd"), p.section("comb"), p.section("kv")
    BM = p.info.q_tile
    # 1) every (query row, key) pair of a segment is covered by exactly one item
    cover = {}
    for q0, q1, k0, k1, pb, seg, s, ns in fwd.tolist():
        assert cq[seg] <= q0 < q1 <= cq[seg + 1] and q1 - q0 <= BM
        assert ck[seg] <= k0 <= k1 <= ck[seg + 1]
        assert (q0 - cq[seg]) % BM == 0
        cover.setdefault((q0, q1), []).append((k0, k1, pb, s, ns))
    for seg in range(len(q_lens)):
        for t in range(cq[seg], cq[seg + 1], BM):
            ranges = sorted(cover.pop((t, min(t + BM, cq[seg + 1]))))
            # key slices partition [ck[seg], ck[seg+1])
            assert ranges[0][0] == ck[seg] and ranges[-1][1] == ck[seg + 1]
            for a, b in zip(ranges, ranges[1:]):
                assert a[1] == b[0]
            ns = len(ranges)
            assert all(r[4] == ns for r in ranges)
            assert (ranges[0][2] == -1) == (ns == 1)
    assert not cover
    # 2) split partial rows are disjoint, contiguous per tile, inside n_part_rows
    used = np.zeros(p.info.n_part_rows, dtype=np.int64)
    # the combine launch sizes its grid by the longest combine item
    assert p.info.max_comb_rows == max([q1 - q0 for q0, q1, *_ in comb.tolist()], default=0)
    for q0, q1, pbase, ns, seg, *_ in comb.tolist():
        R = q1 - q0
        slots = sorted((r[4], r[6]) for r in fwd.tolist() if r[0] == q0 and r[1] == q1)
        assert [s for _, s in slots] == list(range(ns))
        assert [b for b, _ in slots] == [pbase + s * R for s in range(ns)]
        used[pbase:pbase + ns * R] += 1
    assert (used == 1).all()
    # 3) key tiles (plain and fused) cover each key once and carry the
    #    segment's query range; a segment is fused iff it has 1..16 queries,
    #    at least one key and D <= 64, and then all of its key tiles are
    #    fused items (a segment without keys stays on the dQ pass, which
    #    writes its zero rows)
    lq = np.diff(cq)
    fused = (lq > 0) & (lq <= 16) & (np.diff(ck) >= 1) & (D <= 64)
    fkv, fcomb = p.section("fkv"), p.section("fcomb")
    keys = np.zeros(int(ck[-1]), dtype=np.int64)
    BK = p.info.k_tile
    for k0, k1, q0, q1, seg, *_ in kv.tolist():
        assert (q0, q1) == (cq[seg], cq[seg + 1]) and not fused[seg]
        assert (k0 - ck[seg]) % BK == 0 and 0 < k1 - k0 <= BK
        keys[k0:k1] += 1
    for k0, k1, q0, q1, seg, *_ in fkv.tolist():
        assert (q0, q1) == (cq[seg], cq[seg + 1]) and fused[seg]
        keys[k0:k1] += 1
    assert (keys == 1).all()
    # 4) longest-first order
    lens = (fwd[:, 3] - fwd[:, 2]).astype(np.int64)
    assert (np.diff(lens) <= 0).all()
    # 5) the dQ pass runs the forward items (and combines) of the segments
    #    that are not fused, in forward order
    dq, dqc = p.section("dq"), p.section("dqc")
    assert dq.tolist() == [r for r in fwd.tolist() if not fused[r[5]]]
    assert dqc.tolist() == [r for r in comb.tolist() if not fused[r[4]]]
    assert p.info.max_dqc_rows == max([r[1] - r[0] for r in dqc.tolist()], default=0)
    # 6) fused partial rows: chunk j of a segment writes rows pbase + j*Lq + r,
    #    the chunks of all fused segments tile [0, n_fpart_rows) exactly once
    assert sorted(r[4] for r in fcomb.tolist()) == [s for s in range(len(q_lens))
                                                     if fused[s] and k_lens[s] > 0]
    fused_used = np.zeros(p.info.n_fpart_rows, dtype=np.int64)
    tiles = {}
    CH = 3 * 128  # a fused item walks a chunk of three 128-key tiles
    for k0, k1, q0, q1, seg, pbase, j, nt in fkv.tolist():
        assert k0 == ck[seg] + CH * j and nt == -(-int(k_lens[seg]) // CH)
        assert k1 == min(k0 + CH, ck[seg + 1])
        tiles.setdefault(seg, []).append((j, pbase))
    for q0, q1, pbase, nt, seg, *_ in fcomb.tolist():
        R = q1 - q0
        assert sorted(tiles[seg]) == [(j, pbase + j * R) for j in range(nt)]
        fused_used[pbase:pbase + nt * R] += 1
    assert (fused_used == 1).all()
    assert p.info.max_fcomb_rows == max([r[1] - r[0] for r in fcomb.tolist()], default=0)
    return p


def test_varlen_plan_small_cases():
    cases = [([7, 11], [19, 5]), ([129, 257], [33, 130]), ([500, 500], [19, 800]),
             ([512, 512], [500, 500]), ([400], [400]), ([256, 256], [128, 128]),
             ([0, 5, 0], [3, 0, 9]), ([300, 20], [9000, 70000]), ([16, 3], [32768, 1024]),
             ([16, 17, 1], [5000, 5000, 0]), ([64, 2], [129, 128])]
    for ql, kl in cases:
        for D in (32, 64, 128, 256):
            check_varlen_plan(ql, kl, D=D)


def expected_tiles(q_lens, k_lens, D):
    """256-row query tiles for D <= 128 and 256-key tiles for D = 128 when at
    least half of the work (sum of Lq * Lk) lies in segments longer than 128
    queries (keys); 128 otherwise."""
    lq, lk = np.asarray(q_lens, dtype=np.float64), np.asarray(k_lens, dtype=np.float64)
    w = lq * lk
    work = w.sum()
    q = 256 if D <= 128 and work > 0 and 2 * w[lq > 128].sum() >= work else 128
    k = 256 if D == 128 and work > 0 and 2 * w[lk > 128].sum() >= work else 128
    return q, k


def expected_xcd_heads(q_lens, k_lens):
    """Forward grid with an item's heads on one XCD when most of the work lies
    in segments of at most 128 queries."""
    lq, lk = np.asarray(q_lens, dtype=np.float64), np.asarray(k_lens, dtype=np.float64)
    w = lq * lk
    return int(w.sum() > 0 and 2 * w[lq > 128].sum() < w.sum())


@pytest.mark.parametrize("q_lens,k_lens", [
    ([200, 300], [150, 250]),        # long segments: wide tiles at D <= 128 / D = 128
    ([3, 16, 1], [5000, 900, 40]),   # decode-shaped: 128-row tiles, 256-key tiles at D=128
    ([100, 129], [100, 129]),        # 129 * 129 > 100 * 100: the longer segment decides
    ([129, 100, 100], [10, 200, 200]),
    ([0, 0], [5, 7]),                # no work: narrow tiles
    ([300], [64]),                   # long queries, short keys
])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_varlen_tile_choice(q_lens, k_lens, D):
    p = check_varlen_plan(q_lens, k_lens, H=2, D=D)
    assert (p.info.q_tile, p.info.k_tile) == expected_tiles(q_lens, k_lens, D)
    assert p.info.xcd_heads == expected_xcd_heads(q_lens, k_lens)


def test_varlen_tile_choice_on_configs():
    from varlenabsorbflashattn_amd import workloads as W
    c2, c3 = W.config2(0), W.config3(0)
    assert expected_tiles(c2.q_lens, c2.k_lens, c2.D) == (256, 256)
    assert expected_tiles(c3.q_lens, c3.k_lens, c3.D) == (128, 256)
    assert expected_xcd_heads(c2.q_lens, c2.k_lens) == 0
    assert expected_xcd_heads(c3.q_lens, c3.k_lens) == 1


def test_varlen_plan_split_counts_match_reference_rule():
    # prefill-like tiles split ceil(Lk/4096) ways like fa/chunk_indices.py:172-287
    # (per query tile of the plan's height)
    ql, kl = [300, 200, 40], [9000, 4096, 70000]
    for D in (64, 256):  # 256-row tiles at D=64, 128-row tiles at D=256
        p = check_varlen_plan(ql, kl, D=D)
        BM = int(p.info.q_tile)
        assert BM == (256 if D == 64 else 128)
        _, split, comb = meta.split_plan(_cu(ql), _cu(kl), BM, 4096, 4096)
        n_tiles = sum(-(-q // BM) for q in ql)
        assert p.info.n_comb == comb.shape[0]
        assert p.info.n_fwd - (n_tiles - comb.shape[0]) == split.shape[0]


def test_varlen_plan_decode_split_range():
    # Lq <= 16 against >= 1024 keys: 4..16 key chunks per tile
    rng = np.random.default_rng(0)
    lq = rng.integers(1, 17, size=64).tolist()
    lk = rng.integers(1024, 32769, size=64).tolist()
    p = check_varlen_plan(lq, lk, H=32, D=128)
    ns = p.section("comb")[:, 3]
    assert ns.min() >= 4 and ns.max() <= 16 and len(ns) == 64


def test_varlen_plan_stage1_shapes():
    for row in _stage1_cases()[:3]:
        check_varlen_plan(row["q_lens"], row["k_lens"])


def check_absorb_plan(q_lens, k_lens, H=8):
    cq, ck = _cu(q_lens), _cu(k_lens)
    p = _lib.plan_absorb(cq, ck, H, 256, 32)
    TT = p.info.q_tile
    assert TT * H <= 128
    cover = {}
    fwd = p.section("fwd").tolist()
    slot_of = {}
    for pos, (t0, t1, k0, k1, pb, seg, s, ns) in enumerate(fwd):
        if seg == -1:  # no-op slot of the XCD-aware layout
            assert t0 == t1
            continue
        assert cq[seg] <= t0 < t1 <= cq[seg + 1] and t1 - t0 <= TT
        cover.setdefault((t0, t1), []).append((k0, k1))
        # all tiles reading one key range run on one XCD (grid slot mod 8)
        slot_of.setdefault((seg, k0, k1), set()).add(pos % 8)
    assert all(len(v) == 1 for v in slot_of.values())
    for ranges in cover.values():
        ranges.sort()
        for a, b in zip(ranges, ranges[1:]):
            assert a[1] == b[0]
    qt = p.section("qt")
    n_tiles = sum(-(-int(L) // TT) for L in q_lens)
    assert len(qt) == n_tiles == len(cover)
    for t0, t1, k0, k1, pb, seg, *_ in qt.tolist():
        r = sorted(cover[(t0, t1)])
        assert r[0][0] == k0 == ck[seg] and r[-1][1] == k1 == ck[seg + 1]
    comb = p.section("comb").tolist()
    assert p.info.max_comb_rows == max([t1 - t0 for t0, t1, *_ in comb], default=0)
    keys = np.zeros(int(ck[-1]), dtype=np.int64)
    for k0, k1, t0, t1, seg, *_ in p.section("kv").tolist():
        keys[k0:k1] += 1
        assert (t0, t1) == (cq[seg], cq[seg + 1])
    assert (keys == 1).all()
    return p


def test_absorb_plan_cases():
    for ql, kl in [([4], [64]), ([7, 8, 6, 9], [2048, 1024, 1536, 512]), ([5, 7, 9], [123, 257, 999]),
                   ([33, 65, 129], [256] * 3), ([1, 2, 4, 8], [1, 3, 7, 15]), ([0, 3], [5, 0])]:
        check_absorb_plan(ql, kl)


def test_absorb_plan_real_shapes():
    rec = json.load(open(os.path.join(GOLD, "ta_real_shape_subset.json")))["records"][1]
    check_absorb_plan(rec["q_lens"], rec["k_lens"])


def test_plan_rejects_bad_cu():
    with pytest.raises(ValueError):
        _lib.plan_varlen(np.array([0, 5, 3]), np.array([0, 1, 2]), 2, 64)
    with pytest.raises(AssertionError):
        _lib.plan_varlen(np.array([0, 5]), np.array([0, 1, 2]), 2, 64)


def test_host_cu_pair_matches_single_copies():
    import torch
    from varlenabsorbflashattn_amd import _lib
    a = torch.tensor([0, 3, 7, 7, 12], dtype=torch.int32)
    b = torch.tensor([0, 5, 9, 20, 21], dtype=torch.int32)
    for x, y in ((a, a), (a, b), (a, b.to(torch.int64)), (a.numpy(), b)):
        hx, hy = _lib.as_host_i64_pair(x, y)
        assert hx.dtype == np.int64 and hy.dtype == np.int64
        assert np.array_equal(hx, _lib.as_host_i64(x))
        assert np.array_equal(hy, _lib.as_host_i64(y))


def test_absorb_split_chunk_follows_total_work():
    """Key ranges split only beyond a chunk that grows with the launch's total
    work: thousands of samples of <= 8192 keys (configs[3] / configs[4]
    shapes) stay whole, while a handful of very long samples are split into
    chunks of at least 1024 keys so that they fill the GPU."""
    from varlenabsorbflashattn_amd import workloads as W

    def split_counts(ql, kl):
        p = check_absorb_plan(ql, kl)
        fwd = [r for r in p.section("fwd").tolist() if r[5] >= 0]
        return len(fwd), int(p.info.max_split), fwd

    for cfg in (W.config4(seed=0), W.config5(seed=0, n=2048)):
        n, ms, _ = split_counts(cfg.q_lens, cfg.k_lens)
        assert ms == 1, cfg.name
    n, ms, fwd = split_counts([8] * 10, [100000] * 10)
    assert ms > 16 and n == 10 * ms
    assert min(k1 - k0 for _, _, k0, k1, *_ in fwd) >= 1024 - 64
    _, ms, _ = split_counts([5, 9], [40000, 300])
    assert ms == 40  # the many-splits GPU case keeps its 40 chunks


def test_absorb_kv_resident_items_lead():
    """The key-chunk section lists segments with at most 64 (token, head) rows
    first, n_kv_res of them, so the resident-row and streamed dX kernels are
    each launched over only their own items; order within each run is still
    longest-first."""
    H = 8
    q_lens = [1, 8, 9, 0, 20, 3, 8, 100, 2, 9]
    k_lens = [500, 3000, 40, 7, 9000, 1, 260, 129, 64, 5000]
    p = check_absorb_plan(q_lens, k_lens, H=H)
    kv = p.section("kv").tolist()
    n_res = int(p.info.n_kv_res)
    assert len(kv) == int(p.info.n_kv) and 0 < n_res < len(kv)
    rows = [(q1 - q0) * H for (_, _, q0, q1, *_) in kv]
    assert all(r <= 64 for r in rows[:n_res]) and all(r > 64 for r in rows[n_res:])
    up = lambda x, m: (x + m - 1) // m * m
    for run in (kv[:n_res], kv[n_res:]):
        cost = [up(k1 - k0, 128) * up((q1 - q0) * H, 32) for (k0, k1, q0, q1, *_) in run]
        assert cost == sorted(cost, reverse=True)
    # varlen plans have no such split
    assert int(_lib.plan_varlen(_cu([5, 7]), _cu([5, 7]), 2, 64).info.n_kv_res) == 0


# ---- plans of the benchmark configurations ----------------------------------------

def test_config_plans():
    """The plans bench.py runs: C2 needs no key split (L <= 4096); every C3
    (sequence, head) has 4-16 key chunks merged by one combine item, as the
    config prescribes; C4 and C5 keep every sample's key range whole.  Each
    plan also passes the coverage invariants above."""
    from varlenabsorbflashattn_amd import workloads as W
    c2 = W.config2(seed=0)
    p2 = _lib.plan_varlen(_cu(c2.q_lens), _cu(c2.k_lens), c2.H, c2.D)
    assert p2.info.n_comb == 0 and np.all(p2.section("fwd")[:, 4] == -1)
    c3 = W.config3(seed=0)
    p3 = _lib.plan_varlen(_cu(c3.q_lens), _cu(c3.k_lens), c3.H, c3.D)
    fwd, comb = p3.section("fwd"), p3.section("comb")
    assert len(comb) == len(c3.q_lens)          # one query tile per sequence (Lq <= 16)
    assert np.all(fwd[:, 4] >= 0)
    assert 4 <= fwd[:, 7].min() and fwd[:, 7].max() <= 16
    lk = np.asarray(c3.k_lens)
    want = np.clip(-(-lk // 2048), 4, 16)
    assert np.array_equal(comb[np.argsort(comb[:, 4]), 3], want)
    check_varlen_plan(c3.q_lens[:40], c3.k_lens[:40], H=c3.H, D=c3.D)
    for cfg in (W.config4(seed=0), W.config5(seed=0)):
        p = _lib.plan_absorb(_cu(cfg.q_lens), _cu(cfg.k_lens), cfg.H, cfg.D_in, cfg.D_H)
        assert p.info.n_comb == 0 and p.info.max_split == 1, cfg.name


def test_varlen_entry_rejects_plan_of_another_head_dim():
    """A plan with 256-key dK/dV tiles (built for D=128) does not fit the D=64
    kernels: the C ABI refuses it before touching any device memory."""
    import ctypes as C
    cq, ck = _cu([200, 300]), _cu([150, 250])
    p = _lib.plan_varlen(cq, ck, 2, 128)
    assert (p.info.q_tile, p.info.k_tile) == (256, 256)
    lib = _lib.lib()
    rc = lib.vafa_varlen_bwd(None, None, None, None, None, None, None, None, None, None,
                             C.byref(p.info), 64, _lib.DT_BF16, 0.125, None, 0, None)
    assert rc != 0 and "head_dim 64" in _lib.last_error()
    rc = lib.vafa_varlen_fwd(None, None, None, None, None, None, C.byref(p.info), 256,
                             _lib.DT_BF16, 0.0625, None, 0, None)
    assert rc != 0 and "head_dim 256" in _lib.last_error()
    with pytest.raises(ValueError, match="build the plan with this head_dim"):
        _lib.check(rc)


@pytest.mark.parametrize("D", [128, 256])
def test_varlen_bwd_rejects_fused_items_at_wider_head_dim(D):
    """A D=64 plan holds fused key-major items (chunks of up to 3 x 128 keys
    for segments of <= 16 queries); the dK/dV kernels of D=128/256 cover one
    key tile per item, so the C ABI refuses that plan at those head dims
    before any device call (no pointer is dereferenced: all are null)."""
    import ctypes as C
    cq, ck = _cu([5, 100]), _cu([3000, 300])
    p = _lib.plan_varlen(cq, ck, 2, 64)
    assert p.info.n_fkv > 0 and (p.info.q_tile, p.info.k_tile) == (128, 128)
    lib = _lib.lib()
    for stage in (-1, 2):
        if stage < 0:
            rc = lib.vafa_varlen_bwd(None, None, None, None, None, None, None, None, None, None,
                                     C.byref(p.info), D, _lib.DT_BF16, 0.1, None, 0, None)
        else:
            rc = lib.vafa_varlen_bwd_stage(stage, None, None, None, None, None, None, None,
                                           None, None, None, C.byref(p.info), D, _lib.DT_BF16,
                                           0.1, None, 0, None)
        assert rc != 0 and "fused key-major items" in _lib.last_error()
        with pytest.raises(ValueError, match="build the plan with this head_dim"):
            _lib.check(rc)
