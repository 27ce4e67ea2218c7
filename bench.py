"""Benchmark of the two hot operators on one MI355X.

Headline (``value``): packed varlen FlashAttention forward+backward TFLOP/s on
configs[1] (H=16, D=128, bf16, 64 sequences with log-uniform lengths in
[1, 4096], q = k lengths), FLOPs = 4 H D sum(L^2) forward + 10 H D sum(L^2)
backward (fa-tools/benchmark_packed_varlen_flash_attn.py:289-292).  The same
JSON line carries the secondary configurations (split-K forward, absorb
forward GB/s, fp32 and D=256 call shapes), the roofline of the dominant kernel
measured with HIP events on the launch stream, and the CPU baseline (the numpy
oracle on the host cores).  Every timed line reports mean, std, p50, p90, min
and max over its timed iterations, each bracketed by HIP events (the
reference harness's statistics, benchmark_packed_varlen_flash_attn.py:295-313);
the absorb forward lines take their GB/s from the time per call of the same
number of back-to-back calls between one event pair, the reference's absorb
timing (ta/test_smoke.py:629-642).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       python bench.py --only {c2,c2_128k,c3,c4,c4b,c4_fp32,c4full,c5,d16,d256,fused,copy,replay,
                               absorb_shapes,fp32}
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stats(ms):
    """mean / std (population) / p50 / p90 / min / max of a list of ms."""
    xs = sorted(ms)

    def pct(q):
        pos = (len(xs) - 1) * q
        lo, hi = math.floor(pos), math.ceil(pos)
        return xs[lo] + (xs[hi] - xs[lo]) * (pos - lo)

    mean = sum(xs) / len(xs)
    return {"mean": mean, "std": statistics.pstdev(xs) if len(xs) > 1 else 0.0,
            "p50": pct(0.5), "p90": pct(0.9), "min": xs[0], "max": xs[-1], "n": len(xs)}


def timed(fn, iters, warmup=3):
    """Run fn() warmup times (the first calls after a change of workload run
    at a lower shader clock), then iters times with a HIP event pair around
    each call, recorded on torch's current stream (the stream the C ABI
    launches on).  Returns the stats of the per-call ms."""
    import torch
    for _ in range(warmup):
        fn()
    st = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(iters)]
    torch.cuda.synchronize()
    for a, b in evs:
        a.record(st)
        fn()
        b.record(st)
    torch.cuda.synchronize()
    return stats([a.elapsed_time(b) for a, b in evs])


def timed_amortized(fn, iters, warmup=3):
    """ms per call of `iters` back-to-back calls between one HIP event pair,
    the reference's absorb timing (ta/test_smoke.py:629-642).  A per-call
    event pair adds several microseconds to a 0.1 ms call."""
    import torch
    for _ in range(warmup):
        fn()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(st)
    for _ in range(iters):
        fn()
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def timed_both(fn, iters):
    """Per-call stats (timed) plus the amortized ms per call under "amortized"."""
    st = timed(fn, iters)
    st["amortized"] = timed_amortized(fn, iters, warmup=0)
    return st


# ---- varlen -------------------------------------------------------------------

def _varlen_setup(case):
    import torch
    from varlenabsorbflashattn_amd import packed_varlen_attn, workloads as W
    dev = torch.device("cuda:0")
    q, k, v, do = W.varlen_tensors(case, dev, with_grad_out=True)
    cq, ck = W.cu_from_lens(case.q_lens, dev), W.cu_from_lens(case.k_lens, dev)
    q.requires_grad_(True), k.requires_grad_(True), v.requires_grad_(True)

    def step():
        o = packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)
        o.backward(do)
        q.grad = k.grad = v.grad = None

    def fwd():
        with torch.no_grad():
            packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)

    return (q, k, v, do, cq, ck), step, fwd


def bench_varlen_c2(steps, warmup, case=None):
    """C2 fwd+bwd: the contract's wall-clock ms/step over exactly `steps`
    synchronized steps, plus per-step HIP-event stats, the forward alone, and
    the dK/dV kernel (the roofline kernel) timed per launch in the order of a
    training step (forward, delta, dQ, then dK/dV)."""
    import torch
    from varlenabsorbflashattn_amd import workloads as W
    from varlenabsorbflashattn_amd.varlen import BackwardStages
    case = case or W.config2(seed=0)
    (q, k, v, do, cq, ck), step, fwd = _varlen_setup(case)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    step_st = timed(step, steps, warmup=0)
    fwd_st = timed(fwd, max(steps, 3))
    stages = BackwardStages(q.detach(), k.detach(), v.detach(), do, cq, ck)
    evs = []
    for i in range(max(steps, 3) + 1):
        fwd()
        stages.run(0)
        stages.run(1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        stages.run(2)
        e1.record()
        if i > 0:  # the first round is a warmup
            evs.append((e0, e1))
    torch.cuda.synchronize()
    dkv_st = stats([a.elapsed_time(b) for a, b in evs])
    del stages, q, k, v, do
    torch.cuda.empty_cache()
    return case, ms, step_st, fwd_st, dkv_st


def bench_varlen_case(case, steps, warmup):
    """fwd+bwd per-step stats and forward stats (HIP events)."""
    import torch
    _, step, fwd = _varlen_setup(case)
    step_st = timed(step, steps, warmup=warmup)
    fwd_st = timed(fwd, steps)
    torch.cuda.empty_cache()
    return step_st, fwd_st


def bench_varlen_fp32(steps):
    """fp32 varlen on the fp32 matrix cores (the reference's fp32 call,
    fa/interface.py:163) on C2's lengths, fwd+bwd: H=16 with D=16 (padded to
    32), 64 and 128 (both directions on v_mfma_f32_32x32x2_f32), and H=8,
    D=256 (backward on v_mfma_f32_16x16x4_f32); plus configs[0] itself."""
    import torch
    from varlenabsorbflashattn_amd import workloads as W
    c2 = W.config2(seed=0)
    out = {}
    for H, D in ((16, 16), (16, 64), (16, 128), (8, 256)):
        case = W.VarlenCase(f"c2_lengths_H{H}_D{D}_fp32", c2.q_lens, c2.k_lens, H, D,
                            torch.float32)
        s_st, f_st = bench_varlen_case(case, steps, 3)
        out[case.name] = varlen_line(case, s_st, f_st)
        torch.cuda.empty_cache()
    c1 = W.config1(seed=0)
    s_st, f_st = bench_varlen_case(c1, steps, 3)
    out["configs0_fp32"] = varlen_line(c1, s_st, f_st)
    for k_, v_ in out.items():
        log(k_, v_["fwd_ms"]["mean"], v_.get("fwd_bwd_ms", {}).get("mean"))
    return out


def varlen_line(case, step_st, fwd_st):
    """TFLOP/s on the FA2 convention (forward 4, backward 10 H D sum(Lq Lk));
    for 16-bit inputs also as fractions of the 2.5 PFLOP/s bf16/fp16 peak
    (the backward: step mean minus forward mean)."""
    tot = case.flops_fwd + case.flops_bwd
    line = {"sum_L_q": int(sum(case.q_lens)), "sum_L_k": int(sum(case.k_lens)),
            "n_seq": len(case.q_lens), "H": case.H, "D": case.D,
            "fwd_bwd_ms": step_st, "fwd_bwd_TFLOP/s": tot / (step_st["mean"] * 1e-3) / 1e12,
            "fwd_ms": fwd_st, "fwd_TFLOP/s": case.flops_fwd / (fwd_st["mean"] * 1e-3) / 1e12,
            "bwd_TFLOP/s": case.flops_bwd / ((step_st["mean"] - fwd_st["mean"]) * 1e-3) / 1e12}
    if str(case.dtype) in ("torch.bfloat16", "torch.float16"):
        for key in ("fwd_bwd", "fwd", "bwd"):
            line[key + "_frac"] = line[key + "_TFLOP/s"] / BF16_PEAK_TFLOPS
    return line


def fused_case():
    """64 segments of 16 queries against 8192 keys each, H=4, D=64: the
    backward runs the fused key-major dQ/dK/dV kernel."""
    import torch
    from varlenabsorbflashattn_amd import workloads as W
    return W.VarlenCase("varlen_fused_bwd_lq16", [16] * 64, [8192] * 64, 4, 64, torch.bfloat16)


def fused_bwd_bytes(case):
    """Algorithmic backward bytes: q, o, dO read and dq written per query row
    (plus LSE), k, v read and dk, dv written per key row, 2-byte elements."""
    Tq, Tk = sum(case.q_lens), sum(case.k_lens)
    return float(case.H * case.D * 2 * (4 * Tq + 4 * Tk) + case.H * 4 * Tq)


def bench_varlen_c3(iters):
    import torch
    from varlenabsorbflashattn_amd import packed_varlen_attn, workloads as W
    case = W.config3(seed=0)
    dev = torch.device("cuda:0")
    q, k, v = W.varlen_tensors(case, dev)
    cq, ck = W.cu_from_lens(case.q_lens, dev), W.cu_from_lens(case.k_lens, dev)

    def fwd():
        with torch.no_grad():
            packed_varlen_attn(q, k, v, cu_seqlens_q=cq, cu_seqlens_k=ck)

    st = timed(fwd, iters)
    del q, k, v
    torch.cuda.empty_cache()
    return case, st


def replay_records():
    """Production lengths sampled from the reference's fixtures
    (fa-fix/stage1_shapes.jsonl, ta-fix/real_shape_all.json) into tests/golden."""
    g = os.path.join(ROOT, "tests", "golden")
    with open(os.path.join(g, "stage1_shapes_subset.jsonl")) as f:
        stage1 = [json.loads(line) for line in f if line.strip()]
    with open(os.path.join(g, "ta_real_shape_subset.json")) as f:
        ta = json.load(f)["records"]
    return stage1, ta


def bench_replay(steps, warmup, n_stage1=None, n_ta=None):
    """Varlen fwd / fwd+bwd on the stage-1 serving shapes at H=4, D=64
    (fa-tools/benchmark_packed_varlen_flash_attn.py:900-954) and the absorb
    inner op on the real target-attention shapes, d_q=968, d_kv=216
    (ta/test_smoke.py:467-534), bf16; the first n_stage1 / n_ta records of
    each (all by default)."""
    import torch
    from varlenabsorbflashattn_amd import workloads as W
    stage1, ta = replay_records()
    stage1, ta = stage1[:n_stage1], ta[:n_ta]
    out = {"config": "replay", "stage1_H4_D64": [], "ta_real_dq968_dkv216": []}
    for r in stage1:
        case = W.VarlenCase(r["name"], r["q_lens"], r["k_lens"], 4, 64, torch.bfloat16)
        step_st, fwd_st = bench_varlen_case(case, steps, warmup)
        line = {"name": r["name"], **varlen_line(case, step_st, fwd_st)}
        out["stage1_H4_D64"].append(line)
        log({k: (v["mean"] if isinstance(v, dict) else v) for k, v in line.items()})
    for r in ta:
        case = W.AbsorbCase(r["tag"], r["q_lens"], r["k_lens"], 8, 32, int(r["d_kv"]),
                            torch.bfloat16)
        f_st = bench_absorb(case, max(steps, 3), d_q=int(r["d_q"]))
        b_st, _ = bench_absorb_bwd(case, max(steps, 3), d_q=int(r["d_q"]))
        gbs = case.bytes_fwd() / (f_st["amortized"] * 1e-3) / 1e9
        out["ta_real_dq968_dkv216"].append({
            "name": r["tag"], "samples": len(r["q_lens"]), "sum_lq": int(sum(r["q_lens"])),
            "sum_lk": int(sum(r["k_lens"])), "fwd_ms": f_st, "fwd_GB/s": gbs,
            "fwd_hbm_frac": gbs / HBM_PEAK_GBS, "fwd_bwd_ms": b_st})
        log(out["ta_real_dq968_dkv216"][-1]["name"], f_st["mean"], b_st["mean"])
    return out


# ---- absorb --------------------------------------------------------------------

def _absorb_setup(case, d_q=None, dtype=None):
    import torch
    from varlenabsorbflashattn_amd import prepare_target_attn_indices
    from varlenabsorbflashattn_amd import workloads as W
    from varlenabsorbflashattn_amd.absorb import _project_u
    dev = torch.device("cuda:0")
    q_raw, X, W_Q, W_K, W_V = W.absorb_tensors(case, dev, d_q=d_q, dtype=dtype)
    cq, ck = W.cu_from_lens(case.q_lens, dev), W.cu_from_lens(case.k_lens, dev)
    with torch.no_grad():
        u = _project_u(q_raw, W_Q, W_K).contiguous()
    qi, ki = prepare_target_attn_indices(cq, ck)
    return q_raw, X, W_Q, W_K, W_V, u, cq, ck, qi, ki


def bench_absorb(case, iters, d_q=None, full=False, dtype=None):
    """Inner absorb forward on precomputed u, through the reference's hot-path
    contract: prepare_target_attn_indices once, then validate=False calls
    (ta/interface.py:125-138) -- no host round trip inside the timed loop.
    With ``full``, also times the whole packed_target_attn forward on the
    same inputs (16-bit: q_proj, then the attention with u formed inside the
    kernel) and the unfused whole op (projection kernels write u, then the
    inner op reads it); returns (inner, full, unfused) stats."""
    import torch
    from varlenabsorbflashattn_amd import packed_target_attn, target_attn_inner
    from varlenabsorbflashattn_amd.absorb import _project_u
    q_raw, X, W_Q, W_K, W_V, u, cq, ck, qi, ki = _absorb_setup(case, d_q, dtype)
    scale = 1.0 / math.sqrt(case.D_H)

    def fwd():
        with torch.no_grad():
            target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)

    st = timed_both(fwd, iters)
    full_st = None
    if full:
        def full_fwd():
            with torch.no_grad():
                packed_target_attn(q_raw, X, W_Q, W_K, W_V, cu_seqlens_q=cq, cu_seqlens_k=ck,
                                   q_chunk_indices=qi, k_chunk_indices=ki, scale=scale,
                                   validate=False)

        def unfused_fwd():
            with torch.no_grad():
                uu = _project_u(q_raw, W_Q, W_K)
                target_attn_inner(uu, X, W_V, cq, ck, scale, qi, ki, validate=False)

        full_st = timed_both(full_fwd, iters)
        unf_st = timed_both(unfused_fwd, iters)
    del q_raw, X, u
    torch.cuda.empty_cache()
    return (st, full_st, unf_st) if full else st


def bench_absorb_bwd(case, iters, d_q=None, dtype=None):
    """Inner absorb forward + backward (grads of u, X, W_V) on precomputed u,
    validate=False, with a fixed synthetic dO; returns (fwd+bwd, fwd) stats."""
    import torch
    from varlenabsorbflashattn_amd import target_attn_inner
    q_raw, X, W_Q, W_K, W_V, u, cq, ck, qi, ki = _absorb_setup(case, d_q, dtype)
    u.requires_grad_(True)
    X.requires_grad_(True)
    W_V.requires_grad_(True)
    scale = 1.0 / math.sqrt(case.D_H)
    g = torch.Generator().manual_seed(1)
    dO = torch.randn(u.shape[0], case.H, case.D_H, generator=g).to(u.device, u.dtype)

    def step():
        o = target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)
        o.backward(dO)
        u.grad = X.grad = W_V.grad = None

    def fwd():
        with torch.no_grad():
            target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)

    st = timed(step, iters)
    f_st = timed(fwd, iters)
    del q_raw, X, u, dO
    torch.cuda.empty_cache()
    return st, f_st


def bench_absorb_full(case, iters, unfused=False):
    """The whole packed_target_attn (projections included) through the
    prepared-index contract: returns (fwd+bwd, fwd) stats.  With
    ``unfused``, the op is composed of the projection (u written) and the
    inner op instead of taking the folded forward."""
    import torch
    from varlenabsorbflashattn_amd import packed_target_attn, target_attn_inner
    from varlenabsorbflashattn_amd.absorb import _project_u
    q_raw, X, W_Q, W_K, W_V, u, cq, ck, qi, ki = _absorb_setup(case)
    ins = [t.detach().clone().requires_grad_(True) for t in (q_raw, X, W_Q, W_K, W_V)]
    g = torch.Generator().manual_seed(1)
    dO = torch.randn(u.shape[0], case.H, case.D_H, generator=g).to(u.device, u.dtype)

    def call():
        if unfused:
            uu = _project_u(ins[0], ins[2], ins[3])
            return target_attn_inner(uu, ins[1], ins[4], cq, ck, None, qi, ki, validate=False)
        return packed_target_attn(*ins, cu_seqlens_q=cq, cu_seqlens_k=ck, q_chunk_indices=qi,
                                  k_chunk_indices=ki, validate=False)

    def step():
        call().backward(dO)
        for t in ins:
            t.grad = None

    def fwd():
        with torch.no_grad():
            call()

    st = timed(step, iters)
    f_st = timed(fwd, iters)
    del ins, q_raw, X, u, dO
    torch.cuda.empty_cache()
    return st, f_st


def bench_absorb_shapes(iters):
    """The absorb inner op on C4's lengths at the reference's other accepted
    shapes (ta/interface.py:176, 200-201), each on its matrix-core path:
    H = 16 and H = 6 (not dividing 64), D_H = 256, and D_KV = 512 (the FP = 512
    kernels), in bf16; and H = 16 and D_KV = 512 in fp32 (the fp32 matrix-core
    kernels; GB/s counts 4-byte elements there).
    Returns {name: line}."""
    import torch
    from varlenabsorbflashattn_amd import workloads as W
    c4 = W.config4(seed=0)
    out = {}
    bf, f32 = torch.bfloat16, torch.float32
    for H, DH, F, bwd, dt in ((16, 16, 256, True, bf), (6, 32, 96, True, bf),
                              (8, 256, 256, True, bf), (8, 32, 512, True, bf),
                              (16, 16, 256, True, f32), (8, 32, 512, True, f32)):
        tag = "_fp32" if dt == f32 else ""
        case = W.AbsorbCase(f"c4_lengths_H{H}_DH{DH}_F{F}{tag}", c4.q_lens, c4.k_lens, H, DH,
                            F, dt)
        st = bench_absorb(case, iters)
        line = absorb_line(case, st)
        if bwd:
            b_st, _ = bench_absorb_bwd(case, iters)
            line["fwd_bwd_ms"] = b_st
        out[case.name] = line
        log(case.name, st["mean"], line["GB/s"], line.get("fwd_bwd_ms", {}).get("mean"))
    return out


def absorb_line(case, st, full_st=None, unf_st=None):
    """GB/s on the amortized ms per call (back-to-back calls between one event
    pair, ta/test_smoke.py:629-642); GB/s_events and GB/s_p50 on the per-call
    event pairs' mean and median."""
    ms = st.get("amortized", st["mean"])
    gbs = case.bytes_fwd() / (ms * 1e-3) / 1e9
    out = {"ms": st, "GB/s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
           "GB/s_events": case.bytes_fwd() / (st["mean"] * 1e-3) / 1e9,
           "GB/s_p50": case.bytes_fwd() / (st["p50"] * 1e-3) / 1e9,
           "TFLOP/s": case.flops_fwd / (ms * 1e-3) / 1e12,
           "sum_lq": int(sum(case.q_lens)), "sum_lk": int(sum(case.k_lens))}
    if full_st is not None:
        out["packed_target_attn_ms"] = full_st
    if unf_st is not None:
        out["packed_target_attn_unfused_ms"] = unf_st
    return out


# ---- measurement support --------------------------------------------------------

def roofline_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (profiles/roofline_traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "roofline_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("varlen_dkv_kernel", {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _cpu_topology():
    """lscpu's model, sockets, cores per socket, threads per core and CPU
    count, plus the CPUs this process may run on."""
    import subprocess
    out = {}
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        keys = {"Model name": "model", "Socket(s)": "sockets",
                "Core(s) per socket": "cores_per_socket", "Thread(s) per core": "threads_per_core",
                "CPU(s)": "cpus", "NUMA node(s)": "numa_nodes"}
        for line in text.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keys and keys[k.strip()] not in out:
                v = v.strip()
                out[keys[k.strip()]] = int(v) if v.isdigit() else v
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        out["affinity_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    return out


def _blas_threads():
    try:
        import threadpoolctl
        info = [i for i in threadpoolctl.threadpool_info() if i.get("user_api") == "blas"]
        if info:
            return int(info[0]["num_threads"])
    except Exception:  # noqa: BLE001 - reporting only
        pass
    return None


def _median_runs(fn, runs=3):
    fn()  # warmup
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), ts


def cpu_baseline():
    """The reference's CPU path restated (the numpy oracle, fp32) on the host
    cores: 1 warmup + the median of 3 timed runs of each leg.
      * varlen: forward + backward over all 64 segments of C2 (the workload
        itself, fa/test_smoke.py:29-164), reported as TFLOP/s;
      * absorb: the absorbed forward (ta/test_smoke.py:188-229) and the
        explicit-K/V forward (ta/test_smoke.py:111-147) over the first 512 of
        C4's 2048 samples, reported as GB/s of the same algorithmic bytes as
        the GPU line (the reference's torch explicit/absorbed baselines,
        ta/test_smoke.py:1353-1407)."""
    import numpy as np
    import torch
    from oracle import absorb as oa
    from oracle import varlen as ov
    from varlenabsorbflashattn_amd import workloads as W
    case = W.config2(seed=0)
    H, D = case.H, case.D
    rng = np.random.default_rng(0)
    T = sum(case.q_lens)
    q, k, v, do = (rng.standard_normal((T, H, D), dtype=np.float32) for _ in range(4))
    cu = np.zeros(len(case.q_lens) + 1, dtype=np.int64)
    cu[1:] = np.cumsum(case.q_lens)
    sc = 1.0 / math.sqrt(D)

    def varlen_leg():
        ov.forward(q, k, v, cu, cu, sc)
        ov.backward(q, k, v, do, cu, cu, sc)

    v_med, v_runs = _median_runs(varlen_leg)
    flops = case.flops_fwd + case.flops_bwd

    full4 = W.config4(seed=0)
    sub = W.AbsorbCase("c4_first512", full4.q_lens[:512], full4.k_lens[:512], full4.H,
                       full4.D_H, full4.D_in, torch.float32)
    q_raw, X, W_Q, W_K, W_V = (t.numpy() for t in W.absorb_tensors(sub, "cpu"))
    cq = np.concatenate([[0], np.cumsum(sub.q_lens)])
    ck = np.concatenate([[0], np.cumsum(sub.k_lens)])
    asc = 1.0 / math.sqrt(sub.D_H)
    u = oa.project_u(q_raw, W_Q, W_K)
    gpu_bytes = W.AbsorbCase("c4_first512_bf16", sub.q_lens, sub.k_lens, sub.H, sub.D_H,
                             sub.D_in, torch.bfloat16).bytes_fwd()
    a_med, a_runs = _median_runs(lambda: oa.forward(u, X, W_V, cq, ck, asc))
    e_med, e_runs = _median_runs(
        lambda: oa.explicit_forward(q_raw, X, W_Q, W_K, W_V, cq, ck, asc, np.float32))
    return {"value": flops / v_med / 1e12, "unit": "TFLOP/s", "cores": _blas_threads(),
            "kind": "port",
            "sample": f"numpy fp32 oracle forward+backward over all 64 C2 segments "
                      f"(sum L^2 = {int(np.dot(case.q_lens, case.q_lens))}), median of "
                      f"3 runs after 1 warmup: {v_med:.2f} s",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "lscpu": _cpu_topology(),
            "runs_s": v_runs,
            "absorb": {"sample": "first 512 of C4's 2048 samples, fp32 forward",
                       "absorbed_fwd_s": a_med, "absorbed_fwd_GB/s": gpu_bytes / a_med / 1e9,
                       "explicit_fwd_s": e_med, "explicit_fwd_GB/s": gpu_bytes / e_med / 1e9,
                       "note": "GB/s uses the bf16 algorithmic bytes of the GPU line "
                               "(the fp32 CPU run moves twice as many)",
                       "runs_s": {"absorbed": a_runs, "explicit": e_runs}}}


# ---- entry points ---------------------------------------------------------------

def run_only(which, steps, warmup):
    """One configuration, for per-kernel profiling runs."""
    import torch
    from varlenabsorbflashattn_amd import workloads as W
    if which == "copy":
        # calibration for rocprofv3 FETCH_SIZE / WRITE_SIZE: a 1 GiB device copy
        x = torch.empty(1 << 29, dtype=torch.bfloat16, device="cuda:0").fill_(1.0)
        y = torch.empty_like(x)
        st = timed(lambda: y.copy_(x), max(steps, 1))
        return {"config": "copy_1GiB", "ms": st, "GB/s": 2 * (1 << 30) / (st["mean"] * 1e-3) / 1e9}
    if which in ("c2", "c2_128k"):
        case = W.config2(seed=0) if which == "c2" else W.config2_tokens(seed=0)
        case, ms, step_st, fwd_st, dkv_st = bench_varlen_c2(steps, warmup, case)
        return {"config": which, "ms_per_step": ms,
                "TFLOP/s": (case.flops_fwd + case.flops_bwd) / (ms * 1e-3) / 1e12,
                **varlen_line(case, step_st, fwd_st), "dkv_ms": dkv_st}
    if which == "fused":
        case = fused_case()
        step_st, fwd_st = bench_varlen_case(case, max(steps, 3), warmup)
        line = varlen_line(case, step_st, fwd_st)
        line["bwd_GB/s"] = fused_bwd_bytes(case) / ((step_st["mean"] - fwd_st["mean"]) * 1e-3) / 1e9
        return {"config": case.name, **line}
    if which == "d16":
        c = W.config2(seed=0)
        case = W.VarlenCase("c2_lengths_H16_D16", c.q_lens, c.k_lens, 16, 16, torch.bfloat16)
        step_st, fwd_st = bench_varlen_case(case, max(steps, 3), warmup)
        return {"config": case.name, **varlen_line(case, step_st, fwd_st)}
    if which == "d256":
        c = W.config2(seed=0)
        case = W.VarlenCase("c2_lengths_H8_D256", c.q_lens, c.k_lens, 8, 256, torch.bfloat16)
        step_st, fwd_st = bench_varlen_case(case, max(steps, 3), warmup)
        return {"config": case.name, **varlen_line(case, step_st, fwd_st)}
    if which == "c3":
        case, st = bench_varlen_c3(max(steps, 1))
        return {"config": case.name, "ms": st,
                "GB/s": case.bytes_fwd() / (st["mean"] * 1e-3) / 1e9}
    if which == "replay":
        return bench_replay(max(steps, 1), warmup)
    if which == "c4full":
        case = W.config4(seed=0)
        st, f_st = bench_absorb_full(case, max(steps, 1))
        u_st, uf_st = bench_absorb_full(case, max(steps, 1), unfused=True)
        return {"config": case.name + "_packed_target_attn", "fwd_bwd_ms": st, "fwd_ms": f_st,
                "unfused_fwd_bwd_ms": u_st, "unfused_fwd_ms": uf_st}
    if which == "fp32":
        return {"config": "varlen_fp32", **bench_varlen_fp32(max(steps, 3))}
    if which == "absorb_shapes":
        return {"config": "absorb_shapes", **bench_absorb_shapes(max(steps, 3))}
    if which in ("c4b", "c4_fp32"):
        case = W.config4(seed=0)
        dt = torch.float32 if which == "c4_fp32" else None
        st, f_st = bench_absorb_bwd(case, max(steps, 1), dtype=dt)
        return {"config": case.name + ("_fp32" if dt else "") + "_fwd_bwd", "ms": st,
                "fwd_ms": f_st, "bwd_ms": st["mean"] - f_st["mean"]}
    case = W.config4(seed=0) if which == "c4" else W.config5(seed=0)
    st, full_st, unf_st = bench_absorb(case, max(steps, 1), full=True)
    return {"config": case.name, **absorb_line(case, st, full_st, unf_st)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The GPU clock ramps over the first ~15 C2 steps of a process (measured
    # 3.2 -> 2.3 ms per step), so the default warmup runs past that ramp.
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-secondary", action="store_true")
    ap.add_argument("--only", choices=["c2", "c2_128k", "c3", "c4", "c4b", "c4_fp32", "c4full", "c5",
                                       "d16", "d256", "fused", "copy", "replay",
                                       "absorb_shapes", "fp32"],
                    help="run one configuration and print its own JSON line (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the operators have no multi-GPU path "
              "(sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.only:
        print(json.dumps(run_only(args.only, args.steps, args.warmup)))
        return

    case, ms, step_st, fwd_st, dkv_st = bench_varlen_c2(args.steps, args.warmup)
    tflops = (case.flops_fwd + case.flops_bwd) / (ms * 1e-3) / 1e12
    c2 = varlen_line(case, step_st, fwd_st)
    # dK/dV kernel: 4 GEMM passes (S recompute, dP, dV, dK) = 8 H D sum(L^2)
    dkv_flops = 2.0 * case.flops_fwd
    dkv_tflops = dkv_flops / (dkv_st["mean"] * 1e-3) / 1e12
    log(f"C2 fwd+bwd {ms:.3f} ms/step -> {tflops:.1f} TFLOP/s; fwd {fwd_st['mean']:.3f} ms -> "
        f"{c2['fwd_TFLOP/s']:.1f} TFLOP/s; dK/dV kernel {dkv_st['mean']:.3f} ms -> "
        f"{dkv_tflops:.1f} TFLOP/s")
    secondary = {}
    if not args.skip_secondary:
        from varlenabsorbflashattn_amd import workloads as W
        n2 = max(3, args.steps // 2)
        c3, c3_st = bench_varlen_c3(n2)
        gbs = c3.bytes_fwd() / (c3_st["mean"] * 1e-3) / 1e9
        secondary["c3_varlen_splitk_fwd"] = {
            "ms": c3_st, "GB/s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
            "TFLOP/s": c3.flops_fwd / (c3_st["mean"] * 1e-3) / 1e12}
        log("C3", c3_st["mean"], gbs)
        for cfg in (W.config4(seed=0), W.config5(seed=0)):
            # the C4 lines last ~0.1 ms: more iterations for a stable mean
            n_abs = 5 * n2 if cfg.name.startswith("c4") else n2
            st, full_st, unf_st = bench_absorb(cfg, n_abs, full=True)
            secondary[cfg.name + "_fwd"] = absorb_line(cfg, st, full_st, unf_st)
            log(cfg.name, st["mean"], secondary[cfg.name + "_fwd"]["GB/s"])
        c4 = W.config4(seed=0)
        b_st, bf_st = bench_absorb_bwd(c4, 3 * n2)
        p_st, _ = bench_absorb_full(c4, 3 * n2)
        secondary[c4.name + "_fwd_bwd"] = {"ms": b_st, "fwd_ms": bf_st,
                                           "bwd_ms": b_st["mean"] - bf_st["mean"],
                                           "packed_target_attn_fwd_bwd_ms": p_st}
        log(c4.name + " fwd+bwd", b_st["mean"], bf_st["mean"], "full op", p_st["mean"])
        # the reference's documented absorb call is fp32 (no bf16 flag)
        b_st, bf_st = bench_absorb_bwd(c4, n2, dtype=torch.float32)
        c4f = W.AbsorbCase(c4.name, c4.q_lens, c4.k_lens, c4.H, c4.D_H, c4.D_in, torch.float32)
        secondary[c4.name + "_fp32_fwd_bwd"] = {
            "ms": b_st, "fwd_ms": bf_st, "bwd_ms": b_st["mean"] - bf_st["mean"],
            "fwd_GB/s": c4f.bytes_fwd() / (bf_st["mean"] * 1e-3) / 1e9}
        log(c4.name + " fp32 fwd+bwd", b_st["mean"], bf_st["mean"])
        # configs[1] text also says "about 128k total tokens": the same draw
        # extended to 128 Ki tokens
        c2k = W.config2_tokens(seed=0)
        s_st, f_st = bench_varlen_case(c2k, n2, 3)
        secondary["c2_varlen_fwd_bwd_128k_tokens"] = varlen_line(c2k, s_st, f_st)
        log("C2 at 128k tokens", s_st["mean"], f_st["mean"])
        # decode-shaped training backward, where the fused key-major
        # dQ/dK/dV path runs (16 queries per segment, D <= 64)
        cf = fused_case()
        s_st, f_st = bench_varlen_case(cf, n2, 3)
        line = varlen_line(cf, s_st, f_st)
        line["bwd_GB/s"] = fused_bwd_bytes(cf) / ((s_st["mean"] - f_st["mean"]) * 1e-3) / 1e9
        secondary["varlen_fused_bwd_lq16_H4_D64"] = line
        log("fused-path shape", s_st["mean"], f_st["mean"], line["bwd_GB/s"])
        # D=256 (fa/interface.py:167 accepts it) on C2's lengths at H=8
        c256 = W.VarlenCase("c2_lengths_H8_D256", case.q_lens, case.k_lens, 8, 256,
                            torch.bfloat16)
        s_st, f_st = bench_varlen_case(c256, n2, 3)
        secondary["varlen_d256_fwd_bwd"] = varlen_line(c256, s_st, f_st)
        log("D=256", s_st["mean"], f_st["mean"])
        # production replay (the reference's own length fixtures): one stage-1
        # serving record and one real absorb record
        rep = bench_replay(n2, 3, n_stage1=1, n_ta=1)
        secondary["replay_stage1_H4_D64"] = rep["stage1_H4_D64"][0]
        secondary["replay_ta_real_dq968_dkv216"] = rep["ta_real_dq968_dkv216"][0]
        # fp32 varlen on the fp32 matrix cores
        for name, line in bench_varlen_fp32(n2).items():
            secondary["varlen_" + name] = line
        # absorb at the reference's other accepted shapes
        for name, line in bench_absorb_shapes(n2).items():
            secondary["absorb_" + name] = line
        # D=16 (16-bit: the D=32 kernels over zero-padded copies) at C2's shape
        c16 = W.VarlenCase("c2_lengths_H16_D16", case.q_lens, case.k_lens, 16, 16,
                           torch.bfloat16)
        s_st, f_st = bench_varlen_case(c16, n2, 3)
        secondary["varlen_d16_fwd_bwd"] = varlen_line(c16, s_st, f_st)
        log("D=16", s_st["mean"], f_st["mean"])
    cpu = None if args.no_cpu_baseline else cpu_baseline()
    out = {
        "metric": "varlen-FA fwd/bwd TFLOP/s + absorb-attn HBM GB/s, % of MI355X peak",
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[1]: varlen FA fwd+bwd, bf16, H=16, D=128, 64 seqs "
                               "log-uniform[1,4096], q=k lens, non-causal",
                   "seed": 0, "sum_L": int(sum(case.q_lens)),
                   "sum_L2": int(sum(x * x for x in case.q_lens))},
        "step_ms": step_st,
        "roofline": {"bound": "mfma", "kernel": "varlen_dkv_kernel<bf16,128>",
                     "achieved": dkv_tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": dkv_tflops / BF16_PEAK_TFLOPS, "traffic": roofline_traffic(),
                     "work_per_launch": "8*H*D*sum(L^2) = %.4g FLOP" % dkv_flops,
                     "ms_per_launch": dkv_st["mean"], "ms_stats": dkv_st,
                     "timing": "HIP events on the launch stream around each dK/dV launch",
                     "traffic_source": "rocprofv3 FETCH_SIZE x fetch_factor + WRITE_SIZE x "
                                       "write_factor of this kernel on this workload, recorded "
                                       "with the commands in profiles/roofline_traffic.json "
                                       "(bench.py cannot read counters itself)"},
        "c2": c2,
        "secondary": secondary,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
