"""Benchmark of one Token2Tile attention call on one MI355X.

Metric: T2T attention ms/call + TFLOPS at 75.6k tokens,
40 heads, d=128; speedup vs dense.  Workload: the Wan2.1-14B 720p shape
(H=40, N=75600, 1.5% budget, 512 query clusters) on seeded synthetic
Gaussian-mixture inputs in bf16, resident in HBM.

One step = one MaskedStepDeploy.step call under the reuse schedule
mask_refresh=4 (a structure-rebuilding call every 4th step, reuse calls in
between), so ms/step is the R=4-weighted mean.  Full and reuse calls are
also timed separately, per stage, with HIP events on the operator's stream.

Also measured: dense bf16 attention on the same GPU (this library's tile
kernel with an all-ones union, and torch SDPA), the time of a dense call
at the bf16 MFMA peak, init_state cold (first call of the process) and
warm, the roofline fraction of the tile-attention kernel, and the CPU
oracle on the CPU plumbing config over the host cores (at most 16).

A second leg (``profile_max_budget``) re-times the call at the largest
budget the reference's built-in profile for the shape issues (720p: 4880
tokens in the first step window), with its mean union length and the exact
kernel's roofline fraction.

Prints one JSON line.  Usage: python bench.py [--steps K] [--warmup W]
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

MFMA_BF16_PEAK_TFLOPS = 2500.0
# the reference's built-in budget profile for each benchmark shape
# (integrations/sglang/backend/t2t_attn.py:95-130)
PROFILE_FOR = {"wan720p": "wan21_t2v_14b_n75600_t50", "wan480p": "wan21_t2v_n32760_t50"}
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=52)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--config", default="wan720p")
    p.add_argument("--dtype", default="bf16", choices=["bf16", "fp16"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-dense", action="store_true")
    p.add_argument("--no-sdpa", action="store_true", help="skip the torch SDPA dense baseline")
    p.add_argument("--calibrate", action="store_true",
                   help="run one row-permuting copy of K (gather_rows_kernel, known bytes) before "
                        "the warm-up, as the scale reference of FETCH_SIZE/WRITE_SIZE counter runs")
    return p.parse_args()


def traffic_bytes(config, dtype):
    """HBM bytes per launch of the exact attention kernel, from the committed
    FETCH_SIZE / WRITE_SIZE profile of this workload (None when absent)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"attn_kernel_{config}_{dtype}_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def cpu_baseline():
    """The CPU oracle (numpy restatement of the reference semantics) timed
    on one structure-rebuilding call of the CPU plumbing config, with its
    row-parallel stages spread over the host cores this process may use
    (at most 16, the box's CPU share for one GPU), one BLAS thread each."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import parallel as P
    from oracle import t2t_oracle as O
    from token2tile_amd.synth import CONFIGS, budget, generate_np
    H, N, grid, frac, CQ = CONFIGS["cpu_plumbing"]
    q, k, v = generate_np(H, N, grid=grid, seed=0)
    Uq, Uk = O.online_u(q, k, 32)
    Uq, Uk = Uq.astype(np.float16), Uk.astype(np.float16)
    QU, KU = O.project(q, Uq), O.project(k, Uk)
    rng = np.random.default_rng(0)
    st = dict(Uq=Uq, Uk=Uk, ck=KU[:, np.sort(rng.choice(N, 2048, replace=False))],
              cq=QU[:, np.sort(rng.choice(N, CQ, replace=False))])
    cores = min(len(os.sched_getaffinity(0)), 16)
    calls = 3
    with threadpool_limits(limits=1):
        P.full_call_pool(q, k, v, st, budget(N, frac), CQ, workers=cores)   # warm-up
        t0 = time.perf_counter()
        for _ in range(calls):
            P.full_call_pool(q, k, v, st, budget(N, frac), CQ, workers=cores)
        dt = (time.perf_counter() - t0) / calls
    return {"value": round(dt * 1e3, 1), "unit": "ms/call", "cores": cores, "kind": "port",
            "sample": f"mean of {calls} structure-rebuilding calls of the numpy oracle on the CPU "
                      f"plumbing config (H={H}, N={N}, CQ={CQ}, ns={budget(N, frac)}, fp32/fp64), "
                      f"selection, exact attention and merge split over {cores} processes "
                      f"(host cores available: {os.cpu_count()}), one BLAS thread each"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (heads shard "
                                   "across GPUs outside the operator)"}))
        sys.exit(2)
    import torch
    from token2tile_amd import ops
    from token2tile_amd.deploy_step import MaskedStepDeploy
    from token2tile_amd.synth import CONFIGS, budget, generate

    H, N, grid, frac, CQ = CONFIGS[args.config]
    dt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    dev = torch.device("cuda", 0)
    print(f"[bench] config={args.config} H={H} N={N} CQ={CQ} ns={budget(N, frac)} dtype={args.dtype}",
          file=sys.stderr, flush=True)
    q, k, v = generate(H, N, grid=grid, seed=0, device=dev, dtype=dt)
    deploy = MaskedStepDeploy(H, N, CQ, s_frac=frac, mask_refresh=4, device=dev)
    torch.cuda.synchronize()
    # init_state, cold: the first call of the process, which also pays the
    # one-time set-up of the eigensolver and BLAS libraries; warm: a second
    # request on fresh inputs (what every later request and layer pays)
    t0 = time.perf_counter()
    deploy.init_state(*generate(H, N, grid=grid, seed=1, device=dev, dtype=dt)[:2], seed=1)
    torch.cuda.synchronize()
    init_cold_ms = (time.perf_counter() - t0) * 1e3
    t0 = time.perf_counter()
    state = deploy.init_state(q, k, seed=0)
    torch.cuda.synchronize()
    init_ms = (time.perf_counter() - t0) * 1e3
    print(f"[bench] init_state cold {init_cold_ms:.1f} ms, warm {init_ms:.1f} ms", file=sys.stderr,
          flush=True)
    if args.calibrate:
        # reads H*N*256 B of k plus the H*N int32 permutation, writes H*N*256 B
        perm = torch.argsort(torch.rand(H, N, device=dev), dim=1).to(torch.int32)
        ops.fast_gather(k, perm, out=torch.empty_like(k))
        torch.cuda.synchronize()
        del perm

    step_no = [0]

    def one_step(record=None):
        deploy.set_cfg_call(0, key=0, step=step_no[0])
        step_no[0] += 1
        deploy.stage_events = record
        out = deploy.step(q, k, v, state)
        deploy.stage_events = None
        return out

    def timed(steps, warmup):
        """warm-up, then exactly `steps` timed steps; returns ms/step, the
        full / reuse call means and the per-stage means (HIP events on the
        operator's stream, s_main, where every stage kernel is launched)."""
        for _ in range(warmup):
            one_step()
        torch.cuda.synchronize()
        records = []
        t0 = time.perf_counter()
        for _ in range(steps):
            ev = []
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            one_step(ev)
            b.record()
            records.append((deploy.last_call_full, a, b, ev))
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        stages = {"full": {}, "reuse": {}}
        calls = {"full": [], "reuse": []}
        kern = {"attention_exact": [], "attention_residual": []}
        for full, a, b, ev in records:
            kind = "full" if full else "reuse"
            calls[kind].append(a.elapsed_time(b))
            for name, e0, e1 in ev:
                ms = e0.elapsed_time(e1)
                stages[kind].setdefault(name, []).append(ms)
                if name in kern:
                    kern[name].append(ms)
        st_ms = {kd: {n: round(sum(x) / len(x), 4) for n, x in d.items()} for kd, d in stages.items()}
        mean = lambda x: sum(x) / max(1, len(x))
        return wall, mean(calls["full"]), mean(calls["reuse"]), st_ms, {n: mean(x) for n, x in kern.items()}

    def kv_rows():
        snap = deploy._cfg_hold[0]
        pv = ops.plan_views(snap["tile_attn_plan"], H, N, CQ)
        return (pv["kvlen"].long() * snap["tile_sizes"].long()).sum().item()

    wall_ms, full_ms, reuse_ms, stage_ms, kmean = timed(args.steps, args.warmup)
    print(f"[bench] {args.steps} steps: {wall_ms:.3f} ms/step", file=sys.stderr, flush=True)
    print(f"[bench] full {full_ms:.3f} ms, reuse {reuse_ms:.3f} ms, stages {stage_ms}",
          file=sys.stderr, flush=True)
    kern_ms = {"attention_exact": [kmean["attention_exact"]],
               "attention_residual": [kmean["attention_residual"]]}

    # executed attention work: 4 * D * sum_t rows_t * kv_len_t
    snap = deploy._cfg_hold[0]
    rows_kv = kv_rows()
    attn_flops = 4.0 * 128 * rows_kv
    tail_flops = 2.0 * H * N * 2048 * (32 + 128)
    dense_flops = 4.0 * H * N * N * 128
    # the exact-attention kernel (the dominant one) and the residual + merge
    # kernel: average launch duration over the K timed steps
    attn_ms = sum(kern_ms["attention_exact"]) / len(kern_ms["attention_exact"])
    tail_ms = sum(kern_ms["attention_residual"]) / len(kern_ms["attention_residual"])
    attn_tflops = attn_flops / (attn_ms * 1e-3) / 1e12
    tail_tflops = tail_flops / (tail_ms * 1e-3) / 1e12
    value = wall_ms

    # second leg: the largest budget the reference's built-in profile for this
    # shape issues (its first step window), where the exact attention carries
    # most of an end-to-end denoising step
    peak_leg = None
    prof = PROFILE_FOR.get(args.config)
    if prof is not None and args.steps >= 4:
        from token2tile_amd.backend import t2t_attn as BK
        ns_peak = max(BK._ns_map(BK._WAN_PROFILES[prof], N).values())
        deploy.ns_t.fill_(ns_peak)
        w2, f2, r2, st2, k2 = timed(8, 4)
        rk2 = kv_rows()
        fl2 = 4.0 * 128 * rk2
        peak_leg = {"profile": prof, "budget_tokens": ns_peak, "ms_per_step": round(w2, 4),
                    "full_call_ms": round(f2, 3), "reuse_call_ms": round(r2, 3),
                    "mean_kv_len": round(rk2 / (H * N), 1), "stage_ms": st2,
                    "attn_kernel_ms": round(k2["attention_exact"], 4),
                    "attn_frac": round(fl2 / (k2["attention_exact"] * 1e-3) / 1e12
                                       / MFMA_BF16_PEAK_TFLOPS, 4),
                    "residual_kernel_ms": round(k2["attention_residual"], 4)}
        print(f"[bench] profile max budget {ns_peak}: {peak_leg}", file=sys.stderr, flush=True)
        deploy.ns_t.fill_(budget(N, frac))

    result_dense = {}
    if not args.no_dense:
        # dense baseline 1: this library's tile kernel over an all-ones union
        ones = torch.full((H, CQ, 64), -1, dtype=torch.int32, device=dev)
        plan = ops.tile_plan(snap["tile_sizes"], snap["counts"], ones, N)
        kp = ops.fast_gather(k, snap["kperm"])  # K and V in cluster order for the dense launch
        vp = ops.fast_gather(v, snap["kperm"])
        ao = torch.empty_like(q)
        lse = torch.empty(H, N, device=dev, dtype=torch.float32)
        ops.tile_attn_exact(q, kp, vp, snap["counts"], ones, snap["qperm"], plan,
                            attn_out=ao, lse=lse)
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        reps = 2
        a.record()
        for _ in range(reps):
            ops.tile_attn_exact(q, kp, vp, snap["counts"], ones, snap["qperm"], plan,
                                attn_out=ao, lse=lse)
        b.record()
        torch.cuda.synchronize()
        dense_ms = a.elapsed_time(b) / reps
        result_dense["dense_tile_kernel_ms"] = round(dense_ms, 3)
        result_dense["dense_tile_kernel_tflops"] = round(dense_flops / (dense_ms * 1e-3) / 1e12, 1)
        if not args.no_sdpa:
            qq, kk, vv = (x.unsqueeze(0) for x in (q, k, v))
            torch.nn.functional.scaled_dot_product_attention(qq, kk, vv)
            torch.cuda.synchronize()
            a.record()
            for _ in range(reps):
                torch.nn.functional.scaled_dot_product_attention(qq, kk, vv)
            b.record()
            torch.cuda.synchronize()
            result_dense["dense_sdpa_ms"] = round(a.elapsed_time(b) / reps, 3)
            result_dense["speedup_vs_sdpa"] = round(result_dense["dense_sdpa_ms"] / value, 3)
            del qq, kk, vv
        best_dense = min(v_ for k_, v_ in result_dense.items() if k_.endswith("_ms"))
        result_dense["speedup_vs_dense"] = round(best_dense / value, 3)
    # a dense call at the bf16 MFMA peak: the bound no dense kernel can beat
    dense_peak_ms = dense_flops / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e3
    result_dense["dense_at_peak_ms"] = round(dense_peak_ms, 3)
    result_dense["speedup_vs_dense_at_peak"] = round(dense_peak_ms / value, 3)

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline (oracle, cpu plumbing config)...", file=sys.stderr, flush=True)
        cpu = cpu_baseline()

    out = {
        "metric": "T2T attention ms/call + TFLOPS @75.6k tok, 40 heads, d128; speedup vs dense",
        "value": round(value, 4),
        "unit": "ms/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded Gaussian-mixture Q/K with 3-D positional drift, N(0,1) V)",
        "config": {"workload": f"{args.config}: one T2T attention call, mask_refresh=4 schedule",
                   "heads": H, "tokens": N, "head_dim": 128, "key_clusters": 2048,
                   "query_clusters": CQ, "budget_tokens": budget(N, frac), "rank": 32},
        "full_call_ms": round(full_ms, 3),
        "reuse_call_ms": round(reuse_ms, 3),
        "stage_ms": stage_ms,
        "init_state_ms": {"cold": round(init_cold_ms, 1), "warm": round(init_ms, 1)},
        "effective_tflops": round(dense_flops / (value * 1e-3) / 1e12, 1),
        "executed_tflops": round((attn_flops + tail_flops) / (value * 1e-3) / 1e12, 1),
        "mean_kv_len": round(rows_kv / (H * N), 1),
        **result_dense,
        "roofline": {"bound": "mfma", "kernel": "attn_kernel (exact attention over the unions)",
                     "achieved": round(attn_tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(attn_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "kernel_ms": round(attn_ms, 4),
                     "traffic": traffic_bytes(args.config, args.dtype)},
        "roofline_residual": {"bound": "mfma", "kernel": "resid_kernel (centroid residual + merge)",
                              "achieved": round(tail_tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                              "unit": "TFLOP/s",
                              "frac": round(tail_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                              "kernel_ms": round(tail_ms, 4)},
        "cpu_baseline": cpu,
        "profile_max_budget": peak_leg,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
