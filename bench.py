"""Benchmark of the two hot operators on one MI355X.

Headline (``value``): packed varlen FlashAttention forward+backward TFLOP/s on
configs[1] (H=16, D=128, bf16, 64 sequences with log-uniform lengths in
[1, 4096], q = k lengths), FLOPs = 4 H D sum(L^2) forward + 10 H D sum(L^2)
backward.  The same JSON line carries the secondary configurations (split-K
forward, absorb forward GB/s), the roofline of the dominant kernel measured
with HIP events on the launch stream, and the CPU baseline (the numpy oracle
on a bounded sample of the same workload, timed on the host cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_region(fn, iters, stream=None):
    """Average ms of fn() over iters, with HIP events recorded on the launch stream."""
    import torch
    st = stream or torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(st)
    for _ in range(iters):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


def bench_varlen_c2(steps, warmup):
    import torch
    from varlenabsorbflashattn_amd import packed_varlen_attn, workloads as W
    case = W.config2(seed=0)
    dev = torch.device("cuda:0")
    q, k, v, do = W.varlen_tensors(case, dev, with_grad_out=True)
    cu = W.cu_from_lens(case.q_lens, dev)
    q.requires_grad_(True), k.requires_grad_(True), v.requires_grad_(True)

    def step():
        o = packed_varlen_attn(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu)
        o.backward(do)
        q.grad = k.grad = v.grad = None

    def fwd():
        with torch.no_grad():
            packed_varlen_attn(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    fwd_ms = time_region(fwd, max(steps, 3))
    # dominant kernel: dK/dV, timed with HIP events on the launch stream in the
    # order of a training step (forward, delta, dQ, then dK/dV), so the figure
    # matches what a kernel trace of the step reports
    from varlenabsorbflashattn_amd.varlen import BackwardStages
    stages = BackwardStages(q.detach(), k.detach(), v.detach(), do, cu, cu)
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
    dkv_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    del stages
    flops = case.flops_fwd + case.flops_bwd
    return case, ms, fwd_ms, flops, dkv_ms


def bench_varlen_case(case, steps, warmup):
    """fwd+bwd ms/step (wall clock around synchronized steps) and fwd ms (HIP events)."""
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

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    fwd_ms = time_region(fwd, steps)
    del q, k, v, do
    torch.cuda.empty_cache()
    return ms, fwd_ms


def replay_records():
    """Production lengths sampled from the reference's fixtures
    (fa-fix/stage1_shapes.jsonl, ta-fix/real_shape_all.json) into tests/golden."""
    g = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden")
    with open(os.path.join(g, "stage1_shapes_subset.jsonl")) as f:
        stage1 = [json.loads(line) for line in f if line.strip()]
    with open(os.path.join(g, "ta_real_shape_subset.json")) as f:
        ta = json.load(f)["records"]
    return stage1, ta


def bench_replay(steps, warmup):
    """Varlen fwd / fwd+bwd on the stage-1 serving shapes at H=4, D=64
    (fa-tools/benchmark_packed_varlen_flash_attn.py:900-954) and the absorb
    inner op on the real target-attention shapes, d_q=968, d_kv=216
    (ta/test_smoke.py:467-534), bf16."""
    import torch
    from varlenabsorbflashattn_amd import workloads as W
    stage1, ta = replay_records()
    out = {"config": "replay", "stage1_H4_D64": [], "ta_real_dq968_dkv216": []}
    for r in stage1:
        case = W.VarlenCase(r["name"], r["q_lens"], r["k_lens"], 4, 64, torch.bfloat16)
        ms, fwd_ms = bench_varlen_case(case, steps, warmup)
        out["stage1_H4_D64"].append({
            "name": r["name"], "segments": len(r["q_lens"]), "sum_lq": int(sum(r["q_lens"])),
            "sum_lk": int(sum(r["k_lens"])), "fwd_ms": fwd_ms,
            "fwd_TFLOP/s": case.flops_fwd / (fwd_ms * 1e-3) / 1e12, "fwd_bwd_ms": ms,
            "fwd_bwd_TFLOP/s": (case.flops_fwd + case.flops_bwd) / (ms * 1e-3) / 1e12})
        log(out["stage1_H4_D64"][-1])
    for r in ta:
        case = W.AbsorbCase(r["tag"], r["q_lens"], r["k_lens"], 8, 32, int(r["d_kv"]),
                            torch.bfloat16)
        a_ms = bench_absorb(case, max(steps, 3), d_q=int(r["d_q"]))
        b_ms, bf_ms = bench_absorb_bwd(case, max(steps, 3), d_q=int(r["d_q"]))
        gbs = case.bytes_fwd() / (a_ms * 1e-3) / 1e9
        out["ta_real_dq968_dkv216"].append({
            "name": r["tag"], "samples": len(r["q_lens"]), "sum_lq": int(sum(r["q_lens"])),
            "sum_lk": int(sum(r["k_lens"])), "fwd_ms": a_ms, "fwd_GB/s": gbs,
            "fwd_hbm_frac": gbs / HBM_PEAK_GBS, "fwd_bwd_ms": b_ms})
        log(out["ta_real_dq968_dkv216"][-1])
    return out


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

    fwd()
    ms = time_region(fwd, iters)
    del q, k, v
    torch.cuda.empty_cache()
    return case, ms


def bench_absorb(case, iters, d_q=None, full=False):
    """Inner absorb forward on precomputed u, through the reference's hot-path
    contract: prepare_target_attn_indices once, then validate=False calls
    (ta/interface.py:125-138) -- no host round trip inside the timed loop.
    With ``full``, also times the whole packed_target_attn forward (u
    projection included) on the same inputs; returns (inner ms, full ms)."""
    import torch
    from varlenabsorbflashattn_amd import (packed_target_attn, prepare_target_attn_indices,
                                           target_attn_inner)
    from varlenabsorbflashattn_amd import workloads as W
    from varlenabsorbflashattn_amd.absorb import _project_u
    dev = torch.device("cuda:0")
    q_raw, X, W_Q, W_K, W_V = W.absorb_tensors(case, dev, d_q=d_q)
    cq, ck = W.cu_from_lens(case.q_lens, dev), W.cu_from_lens(case.k_lens, dev)
    with torch.no_grad():
        u = _project_u(q_raw, W_Q, W_K).contiguous()
    scale = 1.0 / math.sqrt(case.D_H)
    qi, ki = prepare_target_attn_indices(cq, ck)

    def fwd():
        with torch.no_grad():
            target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)

    fwd()
    ms = time_region(fwd, iters)
    full_ms = None
    if full:
        def full_fwd():
            with torch.no_grad():
                packed_target_attn(q_raw, X, W_Q, W_K, W_V, cu_seqlens_q=cq, cu_seqlens_k=ck,
                                   q_chunk_indices=qi, k_chunk_indices=ki, scale=scale,
                                   validate=False)

        full_fwd()
        full_ms = time_region(full_fwd, iters)
    del q_raw, X, u
    torch.cuda.empty_cache()
    return (ms, full_ms) if full else ms


def bench_absorb_bwd(case, iters, d_q=None):
    """Inner absorb forward + backward (grads of u, X, W_V) on precomputed u,
    validate=False, with a fixed synthetic dO; returns (fwd+bwd ms, fwd ms)."""
    import torch
    from varlenabsorbflashattn_amd import prepare_target_attn_indices, target_attn_inner
    from varlenabsorbflashattn_amd import workloads as W
    from varlenabsorbflashattn_amd.absorb import _project_u
    dev = torch.device("cuda:0")
    q_raw, X, W_Q, W_K, W_V = W.absorb_tensors(case, dev, d_q=d_q)
    cq, ck = W.cu_from_lens(case.q_lens, dev), W.cu_from_lens(case.k_lens, dev)
    with torch.no_grad():
        u = _project_u(q_raw, W_Q, W_K).contiguous()
    u.requires_grad_(True)
    X.requires_grad_(True)
    W_V.requires_grad_(True)
    scale = 1.0 / math.sqrt(case.D_H)
    qi, ki = prepare_target_attn_indices(cq, ck)
    g = torch.Generator().manual_seed(1)
    dO = torch.randn(u.shape[0], case.H, case.D_H, generator=g).to(dev, torch.bfloat16)

    def step():
        o = target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)
        o.backward(dO)
        u.grad = X.grad = W_V.grad = None

    def fwd():
        with torch.no_grad():
            target_attn_inner(u, X, W_V, cq, ck, scale, qi, ki, validate=False)

    step()
    ms = time_region(step, iters)
    f_ms = time_region(fwd, iters)
    del q_raw, X, u, dO
    torch.cuda.empty_cache()
    return ms, f_ms


def roofline_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (profiles/roofline_traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "roofline_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("varlen_dkv_kernel", {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(budget_s=15.0):
    """Oracle (numpy fp32) fwd+bwd on the shortest-first prefix of C2's segments
    that fits the time budget; reported as TFLOP/s of that sample."""
    import numpy as np
    from oracle import varlen as ov
    from varlenabsorbflashattn_amd import workloads as W
    case = W.config2(seed=0)
    rng = np.random.default_rng(0)
    order = np.argsort(case.q_lens)
    done_flops, t_used, n = 0.0, 0.0, 0
    H, D = case.H, case.D
    for i in order:
        L = int(case.q_lens[i])
        q, k, v, do = (rng.standard_normal((L, H, D), dtype=np.float32) for _ in range(4))
        cu = np.array([0, L])
        t0 = time.perf_counter()
        ov.forward(q, k, v, cu, cu, 1.0 / math.sqrt(D))
        ov.backward(q, k, v, do, cu, cu, 1.0 / math.sqrt(D))
        dt = time.perf_counter() - t0
        t_used += dt
        done_flops += 14.0 * H * D * L * L
        n += 1
        if t_used > budget_s:
            break
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": done_flops / t_used / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"numpy fp32 oracle fwd+bwd on the {n} shortest of C2's 64 segments "
                      f"(sum L^2 share {done_flops / (14.0 * H * D * float(np.dot(case.q_lens, case.q_lens))):.3f}), "
                      f"{t_used:.1f} s"}


def run_only(which, steps, warmup):
    """One configuration, for per-kernel profiling runs."""
    from varlenabsorbflashattn_amd import workloads as W
    if which == "copy":
        # calibration for rocprofv3 FETCH_SIZE / WRITE_SIZE: a 1 GiB device copy
        import torch
        x = torch.empty(1 << 29, dtype=torch.bfloat16, device="cuda:0").fill_(1.0)
        y = torch.empty_like(x)
        ms = time_region(lambda: y.copy_(x), max(steps, 1))
        return {"config": "copy_1GiB", "ms": ms, "GB/s": 2 * (1 << 30) / (ms * 1e-3) / 1e9}
    if which == "c2":
        case, ms, fwd_ms, flops, dkv_ms = bench_varlen_c2(steps, warmup)
        return {"config": case.name, "ms_per_step": ms, "TFLOP/s": flops / (ms * 1e-3) / 1e12,
                "fwd_ms": fwd_ms, "dkv_ms": dkv_ms}
    if which == "c3":
        case, ms = bench_varlen_c3(max(steps, 1))
        return {"config": case.name, "ms": ms, "GB/s": case.bytes_fwd() / (ms * 1e-3) / 1e9}
    if which == "replay":
        return bench_replay(max(steps, 1), warmup)
    if which == "c4b":
        case = W.config4(seed=0)
        ms, f_ms = bench_absorb_bwd(case, max(steps, 1))
        return {"config": case.name + "_fwd_bwd", "ms": ms, "fwd_ms": f_ms, "bwd_ms": ms - f_ms}
    case = W.config4(seed=0) if which == "c4" else W.config5(seed=0)
    ms = bench_absorb(case, max(steps, 1))
    return {"config": case.name, "ms": ms, "GB/s": case.bytes_fwd() / (ms * 1e-3) / 1e9}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The GPU clock ramps over the first ~15 C2 steps of a process (measured
    # 3.2 -> 2.3 ms per step), so the default warmup runs past that ramp.
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-secondary", action="store_true")
    ap.add_argument("--only", choices=["c2", "c3", "c4", "c4b", "c5", "copy", "replay"],
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

    case, ms, fwd_ms, flops, dkv_ms = bench_varlen_c2(args.steps, args.warmup)
    tflops = flops / (ms * 1e-3) / 1e12
    fwd_tflops = case.flops_fwd / (fwd_ms * 1e-3) / 1e12
    # dK/dV kernel: 4 GEMM passes (S recompute, dP, dV, dK) = 8 H D sum(L^2)
    dkv_flops = 2.0 * case.flops_fwd
    dkv_tflops = dkv_flops / (dkv_ms * 1e-3) / 1e12
    log(f"C2 fwd+bwd {ms:.3f} ms/step -> {tflops:.1f} TFLOP/s; fwd {fwd_ms:.3f} ms -> "
        f"{fwd_tflops:.1f} TFLOP/s; dK/dV kernel {dkv_ms:.3f} ms -> {dkv_tflops:.1f} TFLOP/s")
    secondary = {}
    if not args.skip_secondary:
        from varlenabsorbflashattn_amd import workloads as W
        c3, c3_ms = bench_varlen_c3(max(3, args.steps // 2))
        secondary["c3_varlen_splitk_fwd"] = {
            "ms": c3_ms, "GB/s": c3.bytes_fwd() / (c3_ms * 1e-3) / 1e9,
            "hbm_frac": c3.bytes_fwd() / (c3_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "TFLOP/s": c3.flops_fwd / (c3_ms * 1e-3) / 1e12}
        log("C3", secondary["c3_varlen_splitk_fwd"])
        for cfg in (W.config4(seed=0), W.config5(seed=0)):
            a_ms, full_ms = bench_absorb(cfg, max(3, args.steps // 2), full=True)
            gbs = cfg.bytes_fwd() / (a_ms * 1e-3) / 1e9
            secondary[cfg.name + "_fwd"] = {
                "ms": a_ms, "GB/s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
                "TFLOP/s": cfg.flops_fwd / (a_ms * 1e-3) / 1e12,
                "packed_target_attn_ms": full_ms,
                "sum_lq": int(sum(cfg.q_lens)), "sum_lk": int(sum(cfg.k_lens))}
            log(cfg.name, secondary[cfg.name + "_fwd"])
        c4 = W.config4(seed=0)
        b_ms, bf_ms = bench_absorb_bwd(c4, max(3, args.steps // 2))
        secondary[c4.name + "_fwd_bwd"] = {"ms": b_ms, "fwd_ms": bf_ms, "bwd_ms": b_ms - bf_ms}
        log(c4.name + " fwd+bwd", secondary[c4.name + "_fwd_bwd"])
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
        "roofline": {"bound": "mfma", "kernel": "varlen_dkv_kernel<bf16,128>",
                     "achieved": dkv_tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": dkv_tflops / BF16_PEAK_TFLOPS, "traffic": roofline_traffic(),
                     "work_per_launch": "8*H*D*sum(L^2) = %.4g FLOP" % dkv_flops,
                     "ms_per_launch": dkv_ms},
        "forward_kernel": {"kernel": "varlen_fwd_kernel<bf16,128>", "ms": fwd_ms,
                           "TFLOP/s": fwd_tflops, "frac": fwd_tflops / BF16_PEAK_TFLOPS},
        "secondary": secondary,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
