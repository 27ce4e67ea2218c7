"""GPU parity of packed_target_attn against the CPU oracle.

Cases follow ta/test_smoke.py:2295-2338 (d_q=968, d_kv=216, H=8, D_H=32,
inputs randn*0.1 as in ta/test_smoke.py:373-395); all five outputs are
compared (O and the grads of q_raw, X, W_Q, W_K, W_V).
"""
import math

import numpy as np
import pytest
import torch

from oracle import absorb as oa
from parity import assert_close
from varlenabsorbflashattn_amd import _lib
from varlenabsorbflashattn_amd import (packed_target_attn, prepare_target_attn_indices,
                                       target_attn_inner)
from varlenabsorbflashattn_amd.workloads import cu_from_lens

pytestmark = pytest.mark.gpu

FP32_CASES = [
    ("smoke", [4], [64]),
    ("single_segment", [7], [256]),
    ("4_uniform", [8, 8, 8, 8], [256] * 4),
    ("4_ragged_real", [7, 8, 6, 9], [2048, 1024, 1536, 512]),
    ("k_tail", [5, 7, 9], [123, 257, 999]),
    ("q_tail", [33, 65, 129], [256, 256, 256]),
    ("short_k_ragged", [1, 2, 4, 8], [1, 3, 7, 15]),
    ("mixed_block_tails", [15, 16, 17, 31], [31, 32, 33, 65]),
    ("nq1_mini", [1], [512]),
]
BF16_CASES = [FP32_CASES[i] for i in (0, 3, 4, 5, 6, 7, 8)] + [
    ("long_split", [3, 40], [5000, 9000]),
    # more key splits (40) than one half-wave combine chunk holds (32)
    ("many_splits", [5, 9], [40000, 300]),
    ("empty_q", [0, 5, 0], [7, 20, 0]),
]


def make_inputs(q_lens, k_lens, d_q=968, d_kv=216, H=8, D_H=32, seed=0):
    g = torch.Generator().manual_seed(seed)
    T_q, T_k = sum(q_lens), sum(k_lens)
    q_raw = torch.randn(T_q, d_q, generator=g) * 0.1
    X = torch.randn(T_k, d_kv, generator=g) * 0.1
    W_Q = torch.randn(d_q, H, D_H, generator=g) * 0.1
    W_K = torch.randn(d_kv, H, D_H, generator=g) * 0.1
    W_V = torch.randn(d_kv, H, D_H, generator=g) * 0.1
    return q_raw, X, W_Q, W_K, W_V


def run_case(q_lens, k_lens, dtype, device, **kw):
    ins = make_inputs(q_lens, k_lens, **kw)
    ins = [t.to(dtype) for t in ins]
    cq, ck = cu_from_lens(q_lens), cu_from_lens(k_lens)
    dev = [t.to(device).requires_grad_(True) for t in ins]
    O = packed_target_attn(*dev, cu_seqlens_q=cq.to(device), cu_seqlens_k=ck.to(device))
    g = torch.Generator().manual_seed(7)
    dO = (torch.randn(O.shape, generator=g) * 0.1).to(dtype)
    O.backward(dO.to(device))
    torch.cuda.synchronize()
    D_H = ins[2].shape[2]
    scale = 1.0 / math.sqrt(D_H)
    npy = [t.float().numpy() for t in ins]
    O_ref = oa.full_forward(*npy, cq.numpy(), ck.numpy(), scale, np.float64)
    grads = oa.full_backward(*npy, dO.float().numpy(), cq.numpy(), ck.numpy(), scale, np.float64)
    return [O] + [t.grad for t in dev], [O_ref] + list(grads)


NAMES = ("O", "dq_raw", "dX", "dW_Q", "dW_K", "dW_V")


@pytest.mark.parametrize("name,q_lens,k_lens", FP32_CASES, ids=[c[0] for c in FP32_CASES])
def test_absorb_fp32_parity(device, name, q_lens, k_lens):
    print(f"[absorb fp32] {name}", flush=True)
    got, ref = run_case(q_lens, k_lens, torch.float32, device)
    for n, a, r in zip(NAMES, got, ref):
        assert_close(n, a, r)


@pytest.mark.parametrize("name,q_lens,k_lens", BF16_CASES, ids=[c[0] for c in BF16_CASES])
def test_absorb_bf16_parity(device, name, q_lens, k_lens):
    print(f"[absorb bf16] {name}", flush=True)
    got, ref = run_case(q_lens, k_lens, torch.bfloat16, device)
    for n, a, r in zip(NAMES, got, ref):
        assert_close(n, a, r)


# head counts and head dims off the benchmark shape (rows of a workgroup are
# laid out head-major, floor(64 / H) tokens per head)
HEAD_SHAPES = [(1, 32, 64), (2, 64, 128), (4, 16, 256), (4, 128, 192), (8, 64, 216),
               # d_kv not a whole number of 16-byte chunks: zero-padded copies
               # (to 56, 104, 512) on the matrix cores
               (2, 16, 50), (8, 32, 100), (3, 16, 509),
               (6, 32, 96),    # H not dividing 64 (10 tokens x 6 heads, 3 heads a wave)
               (16, 32, 128),  # 4 tokens x 16 heads: 4 heads a wave
               (12, 16, 64),   # 5 tokens x 12 heads
               (3, 64, 256),   # 21 tokens x 3 heads
               (5, 256, 192),  # D_H = 256 with H not dividing 64
               (8, 256, 256),  # D_H = 256 at the benchmark width (no fold)
               (10, 32, 256),  # 6 tokens x 10 heads, wide rows (no fold)
               (20, 16, 64),   # 3 tokens x 20 heads: up to 6 heads a wave (no fold)
               (40, 32, 64),   # 1 token x 40 heads, rows 40..63 idle
               (64, 16, 32),   # 1 token x 64 heads: 16 heads a wave
               # 256 < D_KV <= 512: the FP = 512 kernels (16-bit: 2-deep
               # forward ring, du and streamed dX in two f halves on paired
               # workgroups; fp32: du in two halves, dX at one workgroup per CU)
               (8, 32, 384), (4, 64, 512), (2, 16, 264)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("H,D_H,d_kv", HEAD_SHAPES, ids=[f"H{h}_DH{d}_F{f}" for h, d, f in HEAD_SHAPES])
def test_absorb_head_shapes(device, H, D_H, d_kv, dtype):
    """Matrix-core paths (bf16, fp16 and fp32) at head counts, head dims and
    feature widths off the benchmark shape, with the folded projection where
    its kernel takes the shape (at most 4 heads a wave).  d_kv = 50, 100 (16-bit)
    and 509 run on copies zero-padded to a multiple of 8.  D_KV in (256, 512]
    runs on matrix cores in both directions.  The 70-token sample has more than
    64 (token, head) rows, so dX streams its row blocks."""
    print(f"[absorb heads {dtype}] H={H} D_H={D_H} d_kv={d_kv}", flush=True)
    q_lens, k_lens = [1, 9, 70, 3], [40, 300, 129, 2500]
    got, ref = run_case(q_lens, k_lens, dtype, device, d_q=96, d_kv=d_kv, H=H, D_H=D_H)
    for n, a, r in zip(NAMES, got, ref):
        assert_close(n, a, r)


# Heads per wave x D_H >= 128 (16-bit, unfolded) writes aX/l and projects it
# in a row GEMM after the split combine: split key ranges (combined at the
# padded D_KV width, in W_V's re-laid-out f order), padded D_KV (100 -> 104
# -> FP 128), H not dividing 64, and the narrower heads that qualify by
# heads per wave (H = 8, D_H = 64; H = 16, D_H = 32; H = 40, D_H = 16).
WIDE_SPLIT = [(8, 256, 256), (4, 128, 192), (3, 128, 100), (5, 256, 64), (8, 64, 216),
              (16, 32, 128), (40, 16, 64)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("H,D_H,d_kv", WIDE_SPLIT, ids=[f"H{h}_DH{d}_F{f}" for h, d, f in WIDE_SPLIT])
def test_absorb_wide_dh_split(device, H, D_H, d_kv, dtype):
    q_lens, k_lens = [3, 40, 0, 9], [5000, 9000, 4, 70]
    plan = _lib.plan_absorb(cu_from_lens(q_lens).numpy(), cu_from_lens(k_lens).numpy(), H,
                            d_kv, D_H)
    assert plan.info.n_comb > 0, "the case must split a key range"
    print(f"[absorb wide split {dtype}] H={H} D_H={D_H} d_kv={d_kv}", flush=True)
    got, ref = run_case(q_lens, k_lens, dtype, device, d_q=64, d_kv=d_kv, H=H, D_H=D_H)
    for n, a, r in zip(NAMES, got, ref):
        assert_close(n, a, r)


def test_absorb_bf16_config4_dims(device):
    """C4 dims (D_in=256, N(0,1) inputs, Xavier weights) on a small sample."""
    from varlenabsorbflashattn_amd import workloads as W
    case = W.config4(seed=3, n=24)
    q_raw, X, W_Q, W_K, W_V = W.absorb_tensors(case, "cpu")
    cq, ck = cu_from_lens(case.q_lens), cu_from_lens(case.k_lens)
    scale = 1.0 / math.sqrt(case.D_H)
    u = oa.project_u(*(t.float().numpy() for t in (q_raw, W_Q, W_K)), dtype=np.float64)
    u_t = torch.from_numpy(u).to(torch.bfloat16)
    O = target_attn_inner(u_t.to(device), X.to(device), W_V.to(device), cq.to(device),
                          ck.to(device), scale)
    O_ref, _ = oa.forward(u_t.float().numpy(), X.float().numpy(), W_V.float().numpy(),
                          cq.numpy(), ck.numpy(), scale, np.float64)
    assert_close("O", O, O_ref)


@pytest.mark.parametrize("seed,n", [(3, 24), (5, 64)])
def test_absorb_bf16_config4_backward(device, seed, n):
    """Inner backward at C4 dims (D_in=256, H=8, D_H=32, N(0,1) inputs, Xavier
    W_V): grads of u, X and W_V against the fp64 oracle."""
    from varlenabsorbflashattn_amd import workloads as W
    case = W.config4(seed=seed, n=n)
    print(f"[absorb c4 bwd] seed={seed} n={n} sum_lq={sum(case.q_lens)} "
          f"sum_lk={sum(case.k_lens)}", flush=True)
    q_raw, X, W_Q, W_K, W_V = W.absorb_tensors(case, "cpu")
    cq, ck = cu_from_lens(case.q_lens), cu_from_lens(case.k_lens)
    scale = 1.0 / math.sqrt(case.D_H)
    u = oa.project_u(*(t.float().numpy() for t in (q_raw, W_Q, W_K)), dtype=np.float64)
    u_t = torch.from_numpy(u).to(torch.bfloat16)
    g = torch.Generator().manual_seed(seed + 100)
    dO = torch.randn(u_t.shape[0], case.H, case.D_H, generator=g).to(torch.bfloat16)
    dev = [t.to(device).requires_grad_(True) for t in (u_t, X, W_V)]
    O = target_attn_inner(*dev, cq.to(device), ck.to(device), scale)
    O.backward(dO.to(device))
    torch.cuda.synchronize()
    ref = oa.backward(u_t.float().numpy(), X.float().numpy(), W_V.float().numpy(),
                      dO.float().numpy(), cq.numpy(), ck.numpy(), scale, np.float64)
    for name, t, r in zip(("du", "dX", "dW_V"), dev, ref):
        assert_close(name, t.grad, r)


def test_prepared_indices_fast_path(device):
    q_lens, k_lens = [7, 8, 6, 9], [2048, 1024, 1536, 512]
    ins = [t.to(device, torch.bfloat16) for t in make_inputs(q_lens, k_lens)]
    cq, ck = cu_from_lens(q_lens).to(device), cu_from_lens(k_lens).to(device)
    qi, ki = prepare_target_attn_indices(cq, ck)
    from oracle import meta
    assert np.array_equal(qi.cpu().numpy(), meta.chunk_indices(cq.cpu().numpy(), 16))
    assert np.array_equal(ki.cpu().numpy(), meta.chunk_indices(ck.cpu().numpy(), 64))
    a = packed_target_attn(*ins, cu_seqlens_q=cq, cu_seqlens_k=ck)
    b = packed_target_attn(*ins, cu_seqlens_q=cq, cu_seqlens_k=ck, q_chunk_indices=qi,
                           k_chunk_indices=ki, validate=False)
    assert torch.equal(a, b)


def test_prepared_indices_follow_the_call_cu_seqlens(device):
    """Tables prepared for one batch, passed with validate=False alongside the
    cu_seqlens of another batch whose segments have the same block counts but
    other lengths (and larger totals), give that batch's result: the reference
    kernels read the cu_seqlens of each call, so the plan must follow them."""
    q_a, k_a = [7, 8, 6, 9], [200, 100, 150, 64]
    q_b, k_b = [9, 16, 1, 12], [256, 128, 192, 64]   # same ceil(L/16), ceil(L/64)
    ins = [t.to(device, torch.bfloat16) for t in make_inputs(q_b, k_b)]
    cq_a, ck_a = cu_from_lens(q_a).to(device), cu_from_lens(k_a).to(device)
    cq_b, ck_b = cu_from_lens(q_b).to(device), cu_from_lens(k_b).to(device)
    qi, ki = prepare_target_attn_indices(cq_a, ck_a)
    qi_b, ki_b = prepare_target_attn_indices(cq_b, ck_b)
    assert torch.equal(qi, qi_b) and torch.equal(ki, ki_b)
    fresh = packed_target_attn(*ins, cu_seqlens_q=cq_b, cu_seqlens_k=ck_b)
    reused = packed_target_attn(*ins, cu_seqlens_q=cq_b, cu_seqlens_k=ck_b,
                                q_chunk_indices=qi, k_chunk_indices=ki, validate=False)
    assert torch.equal(fresh, reused)
    # an in-place change of the prepared tensors is seen too
    cq_a.copy_(cq_b)
    ck_a.copy_(ck_b)
    again = packed_target_attn(*ins, cu_seqlens_q=cq_a, cu_seqlens_k=ck_a,
                               q_chunk_indices=qi, k_chunk_indices=ki, validate=False)
    assert torch.equal(fresh, again)


def test_prepared_indices_issue_no_device_sync(device):
    """The prepare_target_attn_indices + validate=False contract
    (ta/interface.py:125-138): the host cu_seqlens captured by the prepare
    call are reused, so the inner forward + backward make no synchronizing
    call (torch's sync debug mode turns one into an error)."""
    q_lens, k_lens = [7, 8, 6, 9], [2048, 1024, 1536, 512]
    q_raw, X, W_Q, W_K, W_V = (t.to(device, torch.bfloat16)
                               for t in make_inputs(q_lens, k_lens))
    cq, ck = cu_from_lens(q_lens).to(device), cu_from_lens(k_lens).to(device)
    qi, ki = prepare_target_attn_indices(cq, ck)
    from varlenabsorbflashattn_amd.absorb import _project_u
    u = _project_u(q_raw, W_Q, W_K).contiguous()

    def run():
        uu, xx, ww = (t.detach().clone().requires_grad_(True) for t in (u, X, W_V))
        o = target_attn_inner(uu, xx, ww, cq, ck, None, qi, ki, validate=False)
        o.backward(torch.ones_like(o))
        return o.detach(), uu.grad, xx.grad, ww.grad

    ref = run()  # plan built and cached outside the checked region
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = run()
        # control: without the prepared indices the device cu_seqlens are
        # copied to the host, which the mode catches
        with pytest.raises(RuntimeError):
            target_attn_inner(u, X, W_V, cq, ck, None, validate=False)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_absorb_deterministic(device):
    q_lens, k_lens = [5, 7, 9, 30], [123, 257, 999, 3000]
    outs = []
    for _ in range(2):
        ins = [t.to(device, torch.bfloat16).requires_grad_(True)
               for t in make_inputs(q_lens, k_lens)]
        O = packed_target_attn(*ins, cu_seqlens_q=cu_from_lens(q_lens).to(device),
                               cu_seqlens_k=cu_from_lens(k_lens).to(device))
        O.backward(torch.ones_like(O))
        outs.append([O.detach()] + [t.grad for t in ins])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_absorb_validation_errors(device):
    """The absorb operator's own texts (ta/interface.py:98-116), not the varlen ones."""
    ins = [t.to(device) for t in make_inputs([2, 3], [4, 5])]
    t = lambda *x: torch.tensor(x, device=device)
    cases = [
        (t(0, 2, 5), t(0, 9, 9), "segments with q_len > 0 must have k_len > 0"),
        (t(0, 2, 6), t(0, 4, 9), "cu_seqlens_q[-1] must equal total tokens 5, got 6"),
        (t(1, 2, 5), t(0, 4, 9), "cu_seqlens_q[0] must be 0"),
        (t(0, 4, 3, 5), t(0, 4, 4, 9), "cu_seqlens_q must be non-decreasing"),
        (t(0, 2, 5), t(0, 6, 5, 9)[:3], "cu_seqlens_k[-1] must equal total tokens 9, got 5"),
    ]
    for cq, ck, text in cases:
        with pytest.raises(ValueError) as e:
            packed_target_attn(*ins, cu_seqlens_q=cq, cu_seqlens_k=ck)
        assert str(e.value) == text, (str(e.value), text)
    with pytest.raises(AssertionError, match="segment count mismatch q vs k"):
        packed_target_attn(*ins, cu_seqlens_q=t(0, 2, 5), cu_seqlens_k=t(0, 9))


def test_absorb_bf16_flag_3d_inputs_and_seqinfo(device):
    """packed_target_attn's input forms (ta/interface.py:357-445): bf16=True on
    fp32 inputs, [1, T, d] inputs and seqinfo lengths all give the output of
    the plain call on bf16 inputs with cu_seqlens, bit for bit."""
    q_lens, k_lens = [3, 8, 1], [50, 700, 9]
    ins = make_inputs(q_lens, k_lens)
    cq, ck = cu_from_lens(q_lens).to(device), cu_from_lens(k_lens).to(device)
    b16 = [t.to(torch.bfloat16).to(device) for t in ins]
    base = packed_target_attn(*b16, cu_seqlens_q=cq, cu_seqlens_k=ck)
    flag = packed_target_attn(*(t.to(device) for t in ins), cu_seqlens_q=cq, cu_seqlens_k=ck,
                              bf16=True)
    assert flag.dtype == torch.bfloat16 and torch.equal(flag, base)
    three = packed_target_attn(b16[0].unsqueeze(0), b16[1].unsqueeze(0), *b16[2:],
                               cu_seqlens_q=cq, cu_seqlens_k=ck)
    assert torch.equal(three, base)
    seqinfo = packed_target_attn(*b16, q_seqinfo=torch.tensor(q_lens, device=device),
                                 k_seqinfo=torch.tensor(k_lens, device=device))
    assert torch.equal(seqinfo, base)


def _lib_call(fn, *args):
    from varlenabsorbflashattn_amd import _lib
    _lib.check(getattr(_lib.lib(), fn)(*args))


@pytest.mark.parametrize("T,d_kv,H,D_H", [(9424, 256, 8, 32), (37, 216, 8, 32), (100, 64, 2, 16),
                                          (70, 192, 4, 128), (5, 128, 1, 64), (45, 40, 3, 8),
                                          (33, 64, 2, 256)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_project_u_kernel(device, T, d_kv, H, D_H, dtype):
    """vafa_absorb_project_u (the head einsum of ta/interface.py:435 on matrix
    cores) against a float64 einsum of the same 16-bit inputs: within one
    rounding to the output dtype, token-major [T, H, d_kv] layout."""
    from varlenabsorbflashattn_amd import _lib
    g = torch.Generator().manual_seed(T + d_kv)
    q_proj = torch.randn(T, H * D_H, generator=g).to(dtype)
    W_K = (torch.randn(d_kv, H, D_H, generator=g) * 0.2).to(dtype)
    qd, wd = q_proj.to(device), W_K.to(device)
    u = torch.empty(T, H, d_kv, dtype=dtype, device=device)
    _lib_call("vafa_absorb_project_u", qd.data_ptr(), wd.data_ptr(), u.data_ptr(), T, H, d_kv,
              D_H, _lib.dtype_code(dtype), _lib.stream_ptr(device))
    u = u.cpu()
    ref = torch.einsum("thk,jhk->thj", q_proj.double().view(T, H, D_H), W_K.double())
    err = (u.double() - ref).abs()
    bound = ref.abs() * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10) + 1e-6
    assert (err <= bound).all(), float((err - bound).max())


def _round_bound(ref, absprod, dtype, ulps_in=0.0):
    """|got - ref| allowed for one rounding of a sum to ``dtype`` after fp32
    accumulation: half an output ulp (taken as a relative 2^-8 / 2^-11, with
    a factor 2 of slack), fp32 accumulation error (2^-16 of sum |a_k b_k|: a
    few hundred fp32 additions per output at most, chunk partials included) and,
    where an operand was itself a rounded product, ``ulps_in`` of its ulps
    times sum |a_k b_k|."""
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    return 2 * u * ref.abs() + (2.0 ** -16 + ulps_in * 2 * u) * absprod + 1e-30


PROJECT_SHAPES = [(9424, 256, 256, 8, 32), (37, 968, 216, 8, 32), (1, 96, 64, 2, 16),
                  (130, 40, 192, 4, 128), (0, 64, 64, 2, 32), (300, 72, 8, 3, 8)]


@pytest.mark.parametrize("T,d_q,d_kv,H,D_H", PROJECT_SHAPES,
                         ids=[f"T{s[0]}_dq{s[1]}_dkv{s[2]}_H{s[3]}_DH{s[4]}" for s in PROJECT_SHAPES])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_project_fwd_bwd_kernels(device, T, d_q, d_kv, H, D_H, dtype):
    """vafa_absorb_project_fwd / _bwd through the C ABI against float64
    products of the same 16-bit operands, each product rounded once as the
    reference's 16-bit GEMMs (ta/interface.py:434-435 and torch autograd of
    them): q_proj, u (from the kernel's own q_proj), dq_raw (from the rounded
    float64 dq_proj = du W_K), dW_Q, dW_K; the backward twice with the same
    inputs is bit-identical (deterministic weight gradients)."""
    from varlenabsorbflashattn_amd import _lib
    print(f"[project] T={T} d_q={d_q} d_kv={d_kv} H={H} D_H={D_H} {dtype}", flush=True)
    g = torch.Generator().manual_seed(T * 7 + d_q)
    q_raw = torch.randn(T, d_q, generator=g).to(dtype)
    W_Q = (torch.randn(d_q, H, D_H, generator=g) / math.sqrt(d_q)).to(dtype)
    W_K = (torch.randn(d_kv, H, D_H, generator=g) / math.sqrt(d_kv)).to(dtype)
    du = torch.randn(T, H, d_kv, generator=g).to(dtype)
    HD = H * D_H
    L = _lib.lib()
    code, st = _lib.dtype_code(dtype), _lib.stream_ptr(device)
    qd, wqd, wkd, dud = (t.to(device) for t in (q_raw, W_Q, W_K, du))
    q_proj = torch.empty(T, HD, dtype=dtype, device=device)
    u = torch.empty(T, H, d_kv, dtype=dtype, device=device)
    ws = torch.empty(L.vafa_absorb_project_workspace(T, H, d_q, d_kv, D_H, 0), dtype=torch.uint8,
                     device=device)
    _lib_call("vafa_absorb_project_fwd", qd.data_ptr(), wqd.data_ptr(), wkd.data_ptr(),
              q_proj.data_ptr(), u.data_ptr(), T, H, d_q, d_kv, D_H, code, ws.data_ptr(),
              ws.numel(), st)
    wsb = torch.empty(L.vafa_absorb_project_workspace(T, H, d_q, d_kv, D_H, 1),
                      dtype=torch.uint8, device=device)
    outs = []
    for _ in range(2):
        dq = torch.full((T, d_q), float("nan"), dtype=dtype, device=device)
        dwq = torch.full((d_q, H, D_H), float("nan"), dtype=dtype, device=device)
        dwk = torch.full((d_kv, H, D_H), float("nan"), dtype=dtype, device=device)
        _lib_call("vafa_absorb_project_bwd", qd.data_ptr(), wqd.data_ptr(), wkd.data_ptr(),
                  q_proj.data_ptr(), dud.data_ptr(), dq.data_ptr(), dwq.data_ptr(),
                  dwk.data_ptr(), T, H, d_q, d_kv, D_H, code, wsb.data_ptr(), wsb.numel(), st)
        outs.append([t.cpu() for t in (dq, dwq, dwk)])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    dq, dwq, dwk = outs[0]
    q_proj, u = q_proj.cpu(), u.cpu()

    d = torch.float64
    qr, wq, wk, dd = q_raw.to(d), W_Q.to(d).reshape(d_q, HD), W_K.to(d), du.to(d)
    checks = []
    ref = qr @ wq
    checks.append(("q_proj", q_proj, ref, qr.abs() @ wq.abs(), 0.0))
    qp = q_proj.to(d).view(T, H, D_H)
    ref = torch.einsum("thd,fhd->thf", qp, wk)
    checks.append(("u", u, ref, torch.einsum("thd,fhd->thf", qp.abs(), wk.abs()), 0.0))
    dqp = torch.einsum("thf,fhd->thd", dd, wk).reshape(T, HD)
    dqp_abs = torch.einsum("thf,fhd->thd", dd.abs(), wk.abs()).reshape(T, HD)
    dqp_r = dqp.to(dtype).to(d)
    checks.append(("dq_raw", dq, dqp_r @ wq.t(), dqp_r.abs() @ wq.abs().t(), 1.0))
    checks.append(("dW_Q", dwq.reshape(d_q, HD), qr.t() @ dqp_r, qr.abs().t() @ dqp_abs, 1.0))
    ref = torch.einsum("thf,thd->fhd", dd, qp)
    checks.append(("dW_K", dwk, ref, torch.einsum("thf,thd->fhd", dd.abs(), qp.abs()), 0.0))
    for name, got, ref, absprod, ulps in checks:
        assert got.shape == ref.shape, name
        err = (got.to(d) - ref).abs()
        bound = _round_bound(ref, absprod, dtype, ulps)
        assert torch.isfinite(got).all() and (err <= bound).all(), \
            (name, float((err - bound).max()), float(err.max()))


def test_project_rejects_bad_shapes(device):
    """Unsupported widths and dtypes return an error, and nothing runs."""
    from varlenabsorbflashattn_amd import _lib
    L = _lib.lib()
    assert L.vafa_absorb_project_workspace(16, 2, 60, 64, 32, 0) == -1   # D_Q % 8
    assert L.vafa_absorb_project_workspace(16, 2, 64, 64, 12, 1) == -1   # D_H % 8
    x = torch.zeros(64, dtype=torch.float32, device=device)
    rc = L.vafa_absorb_project_fwd(x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                   x.data_ptr(), 1, 1, 8, 8, 8, _lib.dtype_code(torch.float32),
                                   x.data_ptr(), 256, _lib.stream_ptr(device))
    assert rc != 0 and "16-bit" in _lib.last_error()


# Folded projection (vafa_absorb_fwd_fold): packed_target_attn on 16-bit
# matrix-core shapes forms u inside the attention kernel.  Shapes: the
# benchmark one, one head per wave (H <= 4), D_H = 16 (half the k slots of
# the u product are zero), D_H = 64 / 128 (two / four 32-wide k steps),
# feature widths that pad (216 -> 224, 96 -> 128), and head counts whose
# waves span three or four heads (H = 6: 10 tokens per head; H = 16, 12).
FOLD_SHAPES = [(8, 32, 256), (1, 32, 64), (4, 16, 256), (2, 64, 128), (4, 128, 128),
               (8, 64, 216), (6, 32, 96), (16, 32, 128), (12, 16, 64)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("H,D_H,d_kv", FOLD_SHAPES, ids=[f"H{h}_DH{d}_F{f}" for h, d, f in FOLD_SHAPES])
def test_absorb_fold_matches_unfused_and_oracle(device, H, D_H, d_kv, dtype):
    """The folded forward and its backward against the fp64 oracle, and
    against the unfused path (projection kernel writes u, then
    target_attn_inner) within the same bound.  Lengths hold an empty query
    segment, a split key range (9000 keys) and multi-workgroup samples."""
    from varlenabsorbflashattn_amd.absorb import _fold_native, _project_u
    q_lens, k_lens = [1, 9, 70, 0, 3, 16], [40, 300, 129, 5, 2500, 9000]
    print(f"[absorb fold {dtype}] H={H} D_H={D_H} d_kv={d_kv}", flush=True)
    ins = [t.to(dtype) for t in make_inputs(q_lens, k_lens, d_q=96, d_kv=d_kv, H=H, D_H=D_H)]
    cq, ck = cu_from_lens(q_lens), cu_from_lens(k_lens)
    dev = [t.to(device).requires_grad_(True) for t in ins]
    assert _fold_native(*dev)
    O = packed_target_attn(*dev, cu_seqlens_q=cq.to(device), cu_seqlens_k=ck.to(device))
    g = torch.Generator().manual_seed(7)
    dO = (torch.randn(O.shape, generator=g) * 0.1).to(dtype)
    O.backward(dO.to(device))
    dev2 = [t.to(device).requires_grad_(True) for t in ins]
    u = _project_u(dev2[0], dev2[2], dev2[3])
    O2 = target_attn_inner(u, dev2[1], dev2[4], cq.to(device), ck.to(device))
    O2.backward(dO.to(device))
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(D_H)
    npy = [t.float().numpy() for t in ins]
    O_ref = oa.full_forward(*npy, cq.numpy(), ck.numpy(), scale, np.float64)
    grads = oa.full_backward(*npy, dO.float().numpy(), cq.numpy(), ck.numpy(), scale, np.float64)
    for n, a, b, r in zip(NAMES, [O] + [t.grad for t in dev], [O2] + [t.grad for t in dev2],
                          [O_ref] + list(grads)):
        assert_close(n, a, r)
        assert_close(n + " vs unfused", a, b.detach().float().cpu().numpy())


def test_absorb_fold_negative_scale(device):
    """A negative scale is folded into u as an exact sign flip (before the
    rounding) by the folded kernel, as by the u-reading one."""
    q_lens, k_lens = [3, 8, 1], [50, 700, 3000]
    ins = [t.to(torch.bfloat16) for t in make_inputs(q_lens, k_lens, d_q=64, d_kv=256)]
    cq, ck = cu_from_lens(q_lens), cu_from_lens(k_lens)
    O = packed_target_attn(*(t.to(device) for t in ins), cu_seqlens_q=cq.to(device),
                           cu_seqlens_k=ck.to(device), scale=-0.3)
    npy = [t.float().numpy() for t in ins]
    O_ref = oa.full_forward(*npy, cq.numpy(), ck.numpy(), -0.3, np.float64)
    assert_close("O", O, O_ref)


def test_absorb_fold_prepared_indices_issue_no_device_sync(device):
    """The folded packed_target_attn keeps the prepare_target_attn_indices +
    validate=False contract: forward + backward make no synchronizing call
    and give the validated call's results bit for bit."""
    from varlenabsorbflashattn_amd.absorb import _fold_native
    q_lens, k_lens = [7, 8, 6, 9], [2048, 1024, 1536, 512]
    ins = [t.to(device, torch.bfloat16) for t in make_inputs(q_lens, k_lens)]
    assert _fold_native(*ins)
    cq, ck = cu_from_lens(q_lens).to(device), cu_from_lens(k_lens).to(device)
    qi, ki = prepare_target_attn_indices(cq, ck)

    def run(**kw):
        xs = [t.detach().clone().requires_grad_(True) for t in ins]
        o = packed_target_attn(*xs, cu_seqlens_q=cq, cu_seqlens_k=ck, **kw)
        o.backward(torch.ones_like(o))
        return [o.detach()] + [t.grad for t in xs]

    ref = run()
    run(q_chunk_indices=qi, k_chunk_indices=ki, validate=False)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        got = run(q_chunk_indices=qi, k_chunk_indices=ki, validate=False)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
