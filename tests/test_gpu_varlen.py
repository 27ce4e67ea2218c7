"""GPU parity of packed_varlen_attn against the CPU oracle.

Cases follow fa/test_smoke.py:217-351 (bf16, H=4, D=64 unless noted); the
invariants follow fa/test_smoke.py:354-531.  Tolerances: see tests/parity.py.
"""
import math

import numpy as np
import pytest
import torch

from oracle import varlen as ov
from parity import assert_close, assert_within_reference_numerics, check, report
from varlenabsorbflashattn_amd import packed_varlen_attn, set_validate_cu_seqlens
from varlenabsorbflashattn_amd.workloads import cu_from_lens

pytestmark = pytest.mark.gpu

CASES = [
    ("tiny", [7, 11], [19, 5], 64),
    ("cross_block", [129, 257], [33, 130], 64),
    ("stage1_like", [500, 500], [19, 800], 64),
    ("stage2_like", [512, 512], [500, 500], 64),
    ("single_seg", [400], [400], 64),
    ("block_aligned", [256, 256], [128, 128], 64),
    ("head_dim_128", [200, 300], [150, 250], 128),
    ("head_dim_32", [70, 5], [90, 200], 32),
    # long segments hold most of the work: 256-row query tiles (8-wave forward / dQ)
    ("head_dim_32_wide", [300, 140, 9], [200, 260, 50], 32),
    ("head_dim_16_wide", [260, 20], [300, 3000], 16),
    ("head_dim_256", [130, 3], [77, 300], 256),
    # D=256 dK/dV runs as two workgroups per key tile (one half of d each):
    # several key tiles, a key tail and a split-K forward
    ("head_dim_256_long", [300, 17, 40], [700, 129, 5000], 256),
    ("head_dim_16", [33, 9], [40, 70], 16),
    # D=16 runs on the D=32 matrix-core kernels over zero-padded copies:
    # split-K partials and the fused key-major backward at that width
    ("head_dim_16_split", [3, 40, 129], [5000, 9000, 130], 16),
    ("head_dim_16_fused", [16, 5, 1], [3000, 700, 64], 16),
    ("empty_segments", [0, 5, 9, 0], [3, 0, 40, 7], 64),
    ("long_split", [150, 20], [9000, 5000], 64),
    ("decode_split", [3, 16, 1], [3000, 1500, 1024], 128),
    # more splits than one combine chunk holds (64 per wave row; 32 per
    # half-wave row at D <= 32)
    ("many_splits_d64", [20, 3], [270000, 5000], 64),
    ("many_splits_d32", [20, 7], [140000, 900], 32),
    # fused key-major backward (segments with 1..16 queries at D <= 64): its
    # boundary, key tiles with idle waves (< 32 keys), both head dims it serves
    ("fused_boundary", [16, 17, 1], [5000, 5000, 700], 64),
    ("fused_short_keys", [12, 5, 3], [3, 130, 33], 64),
    ("fused_d32", [16, 2, 40], [600, 4100, 70], 32),
]


def _round_to(dtype):
    """Rounding of an array to ``dtype`` (the kernels' P / dS rounding)."""
    return lambda x: torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dtype) \
        .double().numpy()


def run_case(q_lens, k_lens, H, D, dtype, device, seed=0, dist_scale=1.0, v_scale=1.0,
             reference_numerics=False):
    torch.manual_seed(seed)
    Tq, Tk = sum(q_lens), sum(k_lens)
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(Tq, H, D, generator=g) * dist_scale).to(dtype)
    k = (torch.randn(Tk, H, D, generator=g) * dist_scale).to(dtype)
    v = (torch.randn(Tk, H, D, generator=g) * v_scale).to(dtype)
    do = torch.randn(Tq, H, D, generator=g).to(dtype)
    cq, ck = cu_from_lens(q_lens), cu_from_lens(k_lens)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd = (t.to(device).requires_grad_(True) for t in (q, k, v))
    o = packed_varlen_attn(qd, kd, vd, cu_seqlens_q=cq.to(device), cu_seqlens_k=ck.to(device),
                           scale=scale)
    o.backward(do.to(device))
    torch.cuda.synchronize()
    f64 = np.float64
    o_ref, _ = ov.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), cq.numpy(),
                          ck.numpy(), scale, f64)
    host = [t.float().numpy() for t in (q, k, v, do)]
    dq_r, dk_r, dv_r = ov.backward(*host, cq.numpy(), ck.numpy(), scale, f64)
    got, ref = (o, qd.grad, kd.grad, vd.grad), (o_ref, dq_r, dk_r, dv_r)
    if not reference_numerics:
        return got, ref
    emul = ov.backward(*host, cq.numpy(), ck.numpy(), scale, f64, round_ps=_round_to(dtype))
    return got, ref, emul


@pytest.mark.parametrize("name,q_lens,k_lens,D", CASES, ids=[c[0] for c in CASES])
def test_varlen_bf16_parity(device, name, q_lens, k_lens, D):
    print(f"[varlen bf16] {name} q={q_lens} k={k_lens} D={D}", flush=True)
    got, ref = run_case(q_lens, k_lens, 4, D, torch.bfloat16, device)
    for n, a, r in zip(("o", "dq", "dk", "dv"), got, ref):
        assert_close(n, a, r)


@pytest.mark.parametrize("lens", [
    ([17, 64, 128, 200], [17, 64, 128, 200]),
    # segments of <= 16 queries: the plan routes them to the fused key-major
    # backward (chunks of up to 3 x 128 keys); fp32 runs those chunks on its
    # dK/dV kernel (128-key steps) and their dQ on the pass over forward items
    ([16, 5, 1], [3000, 700, 64]),
], ids=["plain", "fused_planned"])
@pytest.mark.parametrize("D", [64, 16])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["f16", "f32"])
def test_varlen_other_dtypes(device, dtype, D, lens):
    """fp16 and fp32 on the matrix cores (at D=16 over zero-padded D=32
    copies)."""
    print(f"[varlen {dtype}] D={D} q={lens[0]} k={lens[1]}", flush=True)
    got, ref = run_case(lens[0], lens[1], 4, D, dtype, device)
    for n, a, r in zip(("o", "dq", "dk", "dv"), got, ref):
        assert_close(n, a, r)


F32_CASES = [
    ("plain", [17, 64, 128, 200], [17, 64, 128, 200]),
    ("split_k", [150, 20], [9000, 5000]),           # split items + LSE combine
    ("wide_tiles", [300, 140, 9], [200, 260, 50]),  # 256-row query tiles (8 waves)
    ("empty_and_tails", [0, 5, 33, 0], [3, 0, 70, 7]),
    ("decode_split", [3, 16, 1], [3000, 1500, 1024]),
]


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("name,q_lens,k_lens", F32_CASES, ids=[c[0] for c in F32_CASES])
def test_varlen_fp32_matrix_cores(device, name, q_lens, k_lens, D):
    """fp32 on the fp32 matrix cores: forward at D in {32, 64, 128, 256} and
    gradients at D in {32, 64, 128} on v_mfma_f32_32x32x2_f32, D=256 gradients
    on v_mfma_f32_16x16x4_f32, D=16 over zero-padded D=32 copies; against the
    fp64 oracle at the fp32 bound (1e-4 / 1e-5), including split-K partials,
    256-row tiles (walked as two 128-row halves in dQ at D=128), empty
    segments and key tails."""
    print(f"[varlen f32 mfma] {name} q={q_lens} k={k_lens} D={D}", flush=True)
    got, ref = run_case(q_lens, k_lens, 4, D, torch.float32, device)
    for n, a, r in zip(("o", "dq", "dk", "dv"), got, ref):
        assert_close(n, a, r)


def test_varlen_config1_fp32(device):
    """fp32, lens {17,64,128,200}, H=4, D=64 (N(0,1) inputs)."""
    got, ref = run_case([17, 64, 128, 200], [17, 64, 128, 200], 4, 64, torch.float32, device,
                        seed=1)
    assert_close("o", got[0], ref[0])


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dist", [8.0, 0.05])
def test_varlen_input_scales(device, dist, D):
    """Stress distributions of fa-tools/benchmark_packed_varlen_flash_attn.py:226-233
    ("large": inputs x 8, "small": x 0.05), forward and all three gradients as
    that harness checks them (608-615).  At x 8 the scores are 64x larger, so
    the backward's P = exp2(S c - LSE), recomputed from the saved LSE, is
    exercised where it is most sensitive."""
    print(f"[varlen scales] dist={dist} D={D}", flush=True)
    got, ref, emul = run_case([100, 37, 9], [300, 64, 2000], 4, D, torch.bfloat16, device,
                              dist_scale=dist, v_scale=dist, reference_numerics=True)
    # q, k and v are all scaled, as in the harness: at x 8 the softmax is
    # nearly one-hot, so O approaches single V rows (|v| up to ~40) and the
    # gradients carry the x8 of their operands: errors are taken relative to
    # max(1, rms(ref))
    assert_close("o", got[0], ref[0], rel=True)
    for n, a, r, m in zip(("dq", "dk", "dv"), got[1:], ref[1:], emul):
        if dist > 1.0:
            # bounded by the reference algorithm's own rounding of P and dS
            assert_within_reference_numerics(n, a, r, m)
        else:
            assert_close(n, a, r, rel=True)


WIDE_CASES = [
    # (q_lens, k_lens): long segments carry the work, so the plan takes
    # 256-row query tiles, whose forward runs two 32-row blocks per wave
    ([300, 130, 40], [5000, 64, 1]),     # split-K item, Lk = 64, one key
    ([257, 200, 33], [63, 1, 65]),       # first tile is the tail tile; one-row item
    ([520, 3], [700, 2000]),             # three query tiles per (segment, head)
]


@pytest.mark.parametrize("dist", [1.0, 8.0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("case", range(len(WIDE_CASES)))
def test_varlen_wide_tiles(device, case, D, dtype, dist):
    """256-row query tiles (8-wave forward and dQ workgroups) at D = 64 / 128,
    bf16 and fp16: split-K items, one-key and tail-only items, partial waves.
    At dist = 8 (scores scaled 64x, fa-tools/benchmark_packed_varlen_flash_attn.py:226-233)
    later key tiles raise the running max far above the first tile's, so the
    lazy rescale runs on most tiles."""
    from varlenabsorbflashattn_amd import _lib
    q_lens, k_lens = WIDE_CASES[case]
    plan = _lib.plan_varlen(cu_from_lens(q_lens).numpy(), cu_from_lens(k_lens).numpy(), 4, D)
    assert plan.info.q_tile == 256
    print(f"[varlen wide] q={q_lens} k={k_lens} D={D} {dtype} dist={dist}", flush=True)
    got, ref, emul = run_case(q_lens, k_lens, 4, D, dtype, device, dist_scale=dist,
                              reference_numerics=True)
    rel = dist > 1.0  # near one-hot rows: see test_varlen_input_scales
    assert_close("o", got[0], ref[0], rel=rel)
    for name, a, r, m in zip(("dq", "dk", "dv"), got[1:], ref[1:], emul):
        if dist > 1.0:
            assert_within_reference_numerics(name, a, r, m)
        else:
            assert_close(name, a, r)


@pytest.mark.parametrize("H,q_lens,k_lens,D", [
    (3, [300, 5, 140], [200, 3000, 150], 64),     # 256-row tiles, item-major grid
    (5, [3, 16, 1, 9], [3000, 1500, 1024, 40], 128),  # decode-shaped: an item's heads on one XCD
    (7, [130, 20], [5000, 9000], 32),             # split-K items and their combine
])
def test_varlen_odd_head_counts(device, H, q_lens, k_lens, D):
    """Head counts that are not multiples of the 8 XCDs, on both forward grid
    layouts (the plan's xcd_heads flag), forward and backward."""
    from varlenabsorbflashattn_amd import _lib
    plan = _lib.plan_varlen(cu_from_lens(q_lens).numpy(), cu_from_lens(k_lens).numpy(), H, D)
    print(f"[varlen odd H] H={H} q={q_lens} k={k_lens} D={D} xcd_heads={plan.info.xcd_heads}",
          flush=True)
    got, ref = run_case(q_lens, k_lens, H, D, torch.bfloat16, device)
    for name, a, r in zip(("o", "dq", "dk", "dv"), got, ref):
        assert_close(name, a, r)


def test_single_key_returns_v(device):
    """Lk = 1: softmax weight 1 -> O == V exactly; dq = dk = 0 up to fp32 rounding
    (delta = O.dO and dP = dO.V are summed in different orders)."""
    H, D = 2, 64
    q = torch.randn(5, H, D, device=device, dtype=torch.bfloat16, requires_grad=True)
    k = torch.randn(1, H, D, device=device, dtype=torch.bfloat16, requires_grad=True)
    v = torch.randn(1, H, D, device=device, dtype=torch.bfloat16, requires_grad=True)
    o = packed_varlen_attn(q, k, v, cu_seqlens_q=torch.tensor([0, 5], device=device),
                           cu_seqlens_k=torch.tensor([0, 1], device=device))
    assert torch.equal(o, v.expand(5, H, D))
    o.backward(torch.randn_like(o))
    assert q.grad.abs().max().item() < 1e-5 and k.grad.abs().max().item() < 1e-5


def test_one_hot_segment_values(device):
    """V one-hot on the segment id: column seg is ~1, every other column exactly 0."""
    lens = [3, 70, 129, 1, 260]
    H, D = 2, 64
    cu = cu_from_lens(lens).to(device)
    T = sum(lens)
    seg = torch.repeat_interleave(torch.arange(len(lens)), torch.tensor(lens))
    v = torch.zeros(T, H, D)
    v[torch.arange(T), :, seg] = 1.0
    q = torch.randn(T, H, D)
    k = torch.randn(T, H, D)
    o = packed_varlen_attn(*(t.to(device, torch.bfloat16) for t in (q, k, v)),
                           cu_seqlens_q=cu, cu_seqlens_k=cu).float().cpu()
    mask = torch.zeros(T, H, D, dtype=torch.bool)
    mask[torch.arange(T), :, seg] = True
    assert o[~mask].abs().max().item() == 0.0
    assert (o[mask] - 1).abs().max().item() < 1e-2


def _inputs(device, q_lens=(129, 257), k_lens=(33, 130), H=4, D=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    Tq, Tk = sum(q_lens), sum(k_lens)
    q, k, v = (torch.randn(T, H, D, generator=g).to(device, torch.bfloat16)
               for T in (Tq, Tk, Tk))
    return q, k, v, cu_from_lens(q_lens).to(device), cu_from_lens(k_lens).to(device)


def test_no_grad_equals_grad(device):
    q, k, v, cq, ck = _inputs(device)
    with torch.no_grad():
        a = packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)
    b = packed_varlen_attn(q.requires_grad_(), k.requires_grad_(), v.requires_grad_(),
                           cu_seqlens_q=cq, cu_seqlens_k=ck)
    assert torch.equal(a, b.detach())


def test_3d_equals_4d(device):
    q, k, v, cq, ck = _inputs(device)
    outs = []
    for unsq in (False, True):
        qq, kk, vv = (t.detach().clone().unsqueeze(0) if unsq else t.detach().clone()
                      for t in (q, k, v))
        for t in (qq, kk, vv):
            t.requires_grad_(True)
        o = packed_varlen_attn(qq, kk, vv, cu_seqlens_q=cq, cu_seqlens_k=ck)
        assert o.dim() == (4 if unsq else 3)
        o.backward(torch.ones_like(o))
        outs.append([t.squeeze(0) for t in (o.detach(), qq.grad, kk.grad, vv.grad)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_repeatable_bit_exact(device):
    """Two runs with dO = 1 agree bit for bit (no atomics; fa/test_smoke.py:496-531)."""
    q, k, v, cq, ck = _inputs(device, q_lens=(300, 20), k_lens=(9000, 500))
    res = []
    for _ in range(2):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o = packed_varlen_attn(qq, kk, vv, cu_seqlens_q=cq, cu_seqlens_k=ck)
        o.backward(torch.ones_like(o))
        res.append((o.detach(), qq.grad, kk.grad, vv.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_partial_grad(device):
    """Only q requires grad: k.grad / v.grad stay None (fa/test_smoke.py:379-407)."""
    q, k, v, cq, ck = _inputs(device)
    q.requires_grad_(True)
    o = packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)
    o.sum().backward()
    assert q.grad is not None and k.grad is None and v.grad is None


def test_seqinfo_equals_cu_and_validation_toggle(device):
    q, k, v, cq, ck = _inputs(device)
    a = packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)
    b = packed_varlen_attn(q, k, v, q_seqinfo=torch.tensor([129, 257], device=device),
                           k_seqinfo=torch.tensor([33, 130], device=device))
    set_validate_cu_seqlens(False)
    try:
        c = packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)
    finally:
        set_validate_cu_seqlens(True)
    assert torch.equal(a, b) and torch.equal(a, c)
    with pytest.raises(ValueError):
        packed_varlen_attn(q, k, v, cu_seqlens_q=torch.tensor([0, 100, 380], device=device),
                           cu_seqlens_k=ck)


@pytest.mark.parametrize("seed", range(5))
def test_multi_seed(device, seed):
    got, ref = run_case([77, 200, 3], [150, 31, 260], 4, 64, torch.bfloat16, device, seed=seed)
    for n, a, r in zip(("o", "dq", "dk", "dv"), got, ref):
        assert_close(n, a, r)


@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_backward_stages_match_fused(device, D):
    """vafa_varlen_bwd_stage (delta, dQ, dK/dV launched separately) reproduces
    vafa_varlen_bwd, whose dQ kernel forms delta itself, bit for bit."""
    from varlenabsorbflashattn_amd.varlen import BackwardStages
    print(f"[varlen stages] D={D}", flush=True)
    # the 9-query segment is fused-planned at D <= 64 (dQ from the key-major
    # kernel's partials, summed in the dK/dV stage)
    q, k, v, cq, ck = _inputs(device, q_lens=(300, 20, 77, 9), k_lens=(9000, 500, 64, 2000), D=D)
    do = torch.randn_like(q)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o = packed_varlen_attn(qq, kk, vv, cu_seqlens_q=cq, cu_seqlens_k=ck)
    o.backward(do)
    st = BackwardStages(q, k, v, do, cq, ck)
    for s in (0, 1, 2):
        st.run(s)
    torch.cuda.synchronize()
    assert torch.equal(st.o, o.detach())
    assert torch.equal(st.dq, qq.grad) and torch.equal(st.dk, kk.grad) and torch.equal(st.dv, vv.grad)


def test_stage1_real_shape(device):
    """A production stage-1 shape (fa-fix/stage1_shapes.jsonl, sampled into
    tests/golden): 500 queries per user against up to 102400 keys at H=4,
    D=64, so every tile runs the 4096-key split path and the LSE combine."""
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "stage1_shapes_subset.jsonl")
    with open(path) as f:
        rec = json.loads(f.readline())
    q_lens, k_lens = rec["q_lens"][:3], rec["k_lens"][:3]
    print(f"[varlen stage1] {rec['name']} q={q_lens} k={k_lens}", flush=True)
    got, ref = run_case(q_lens, k_lens, 4, 64, torch.bfloat16, device)
    for n, a, r in zip(("o", "dq", "dk", "dv"), got, ref):
        assert_close(n, a, r)


def test_host_cu_seqlens_issue_no_device_sync(device):
    """cu_seqlens held on the host skip the per-call device-to-host copy: the
    plan is looked up from them directly, so a forward + backward makes no
    synchronizing call (torch's sync debug mode turns one into an error), and
    the results equal those of device cu_seqlens bit for bit."""
    q, k, v, cq, ck = _inputs(device, q_lens=(300, 20, 77), k_lens=(9000, 500, 64))
    do = torch.randn_like(q)
    cq_h, ck_h = cq.cpu(), ck.cpu()

    def run(a, b):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        o = packed_varlen_attn(qq, kk, vv, cu_seqlens_q=a, cu_seqlens_k=b)
        o.backward(do)
        return o.detach(), qq.grad, kk.grad, vv.grad

    ref = run(cq, ck)
    run(cq_h, ck_h)  # plan built and cached outside the checked region
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = run(cq_h, ck_h)
        # control: device cu_seqlens are copied to the host, which the mode catches
        with pytest.raises(RuntimeError):
            run(cq, ck)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_noncontiguous_inputs_match_contiguous(device):
    """Non-contiguous q/k/v views (the stress option of
    fa-tools/benchmark_packed_varlen_flash_attn.py:248-253) give the results of
    their contiguous copies bit for bit, and the grads reach the views' bases."""
    q, k, v, cq, ck = _inputs(device, q_lens=(70, 130), k_lens=(90, 300), D=64)
    do = torch.randn_like(q)
    T, H, D = q.shape
    qb = torch.zeros(T, H, 2 * D, device=device, dtype=q.dtype)
    qb[..., ::2] = q                                   # stride(-1) == 2
    kb = k.transpose(0, 1).contiguous()                # view strides (D, T*D, 1)
    vb = torch.cat([v, torch.zeros_like(v)], dim=1)    # view strides (2*H*D, D, 1)
    for t in (qb, kb, vb):
        t.requires_grad_(True)
    views = (qb[..., ::2], kb.transpose(0, 1), vb[:, :H])
    assert not any(t.is_contiguous() for t in views)
    o1 = packed_varlen_attn(*views, cu_seqlens_q=cq, cu_seqlens_k=ck)
    o1.backward(do)
    q2, k2, v2 = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    o2 = packed_varlen_attn(q2, k2, v2, cu_seqlens_q=cq, cu_seqlens_k=ck)
    o2.backward(do)
    assert torch.equal(o1, o2)
    assert torch.equal(qb.grad[..., ::2], q2.grad) and not qb.grad[..., 1::2].any()
    assert torch.equal(kb.grad.transpose(0, 1), k2.grad)
    assert torch.equal(vb.grad[:, :H], v2.grad) and not vb.grad[:, H:].any()


def _gpu_errors(out, ref):
    """The parity.py metrics evaluated on the GPU (for tensors too large to
    move to the host): raw max and mean of |out - ref|, the largest rounding
    of ref to the output dtype, and max(|out - ref| - that rounding)."""
    a, r = out.detach().float(), ref.detach().float()
    floor = (r.to(out.dtype).float() - r).abs()
    d = (a - r).abs()
    return dict(max_abs=d.max().item(), mean_abs=d.mean().item(), floor=floor.max().item(),
                excess=(d - floor).max().item(), rms=r.pow(2).mean().sqrt().item(),
                ref_max=r.abs().max().item())


def test_varlen_business_scale(device):
    """fa/test_smoke.py:666-767: 50 segments x Q=500 against K_total = 2M keys
    with pareto-distributed key lengths (H=4, D=64, bf16), forward and grads
    against a float32 torch reference computed per segment on the GPU."""
    n, Lq, H, D, K_total = 50, 500, 4, 64, 2_000_000
    rng = np.random.default_rng(0)
    w = rng.pareto(1.5, n) + 1.0
    k_lens = np.maximum(1, np.floor(w / w.sum() * K_total)).astype(np.int64)
    k_lens[0] += K_total - int(k_lens.sum())
    q_lens = [Lq] * n
    print(f"[varlen business] n={n} Lq={Lq} K_total={int(k_lens.sum())} max_k={int(k_lens.max())}",
          flush=True)
    g = torch.Generator(device=device).manual_seed(0)
    Tq, Tk = n * Lq, int(k_lens.sum())
    q = torch.randn(Tq, H, D, device=device, generator=g).to(torch.bfloat16)
    k = torch.randn(Tk, H, D, device=device, generator=g).to(torch.bfloat16)
    v = torch.randn(Tk, H, D, device=device, generator=g).to(torch.bfloat16)
    do = torch.randn(Tq, H, D, device=device, generator=g).to(torch.bfloat16)
    cq, ck = cu_from_lens(q_lens).to(device), cu_from_lens(k_lens.tolist()).to(device)
    qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = packed_varlen_attn(qd, kd, vd, cu_seqlens_q=cq, cu_seqlens_k=ck)
    o.backward(do)
    scale = 1.0 / math.sqrt(D)
    torch.backends.cuda.matmul.allow_tf32 = False
    o_r = torch.empty(Tq, H, D, device=device)
    dq_r = torch.empty(Tq, H, D, device=device)
    dk_r = torch.empty(Tk, H, D, device=device)
    dv_r = torch.empty(Tk, H, D, device=device)
    q0 = k0 = 0
    for lk in k_lens.tolist():
        qs, ks, vs = (t.float().transpose(0, 1).contiguous().requires_grad_(True)
                      for t in (q[q0:q0 + Lq], k[k0:k0 + lk], v[k0:k0 + lk]))
        p = torch.softmax(torch.matmul(qs, ks.transpose(1, 2).contiguous()) * scale, dim=-1)
        os_ = torch.matmul(p, vs)
        os_.backward(do[q0:q0 + Lq].float().transpose(0, 1).contiguous())
        o_r[q0:q0 + Lq] = os_.detach().transpose(0, 1)
        dq_r[q0:q0 + Lq] = qs.grad.transpose(0, 1)
        dk_r[k0:k0 + lk] = ks.grad.transpose(0, 1)
        dv_r[k0:k0 + lk] = vs.grad.transpose(0, 1)
        q0 += Lq
        k0 += lk
    for name, a, r in (("o", o, o_r), ("dq", qd.grad, dq_r), ("dk", kd.grad, dk_r),
                       ("dv", vd.grad, dv_r)):
        e = _gpu_errors(a, r)
        report(name, e, torch.bfloat16)
        check(name, e, torch.bfloat16)
