"""Masked-component fwd+bwd throughput on one MI355X.

Default workload: the single decomposed dense linear 768 -> 3072 (x bf16 [4096, 768] ~
N(0,1), U/V ~ N(0, 1/d), C = 4096 components, per-component gate MLP hidden 16 with
leaky-hard-sigmoid squashing, bf16 Threefry mask uniforms, fp32 accumulation, one fused
fwd+bwd of stochastic-recon MSE + sum_c mean_t |g_upper|^2). A step is one call of
`pd_dense_step` on resident inputs: clean target, h = x@V, gate/mask, (h*m)@U, MSE,
imp-min, and the backward to dV, dU and the gate parameters.

Prints one JSON line: the throughput (tokens/s), the roofline of the dominant kernel
(measured with HIP events on the kernels' own stream over the timed region), per-phase
times, and the CPU baseline (the oracle's C restatement, OpenMP, on a bounded token
sample, timed in this run on this host).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_FLOPS = 2.5e15
PEAK_F32_FLOPS = 157.3e12
PEAK_HBM = 8.0e12

WORKLOADS = {
    "dense768x3072_C4096": dict(T=4096, d_in=768, d_out=3072, C=4096),
}
METRIC = "masked-component fwd+bwd tokens/s on 1 MI355X; % of MFMA/HBM roofline"


def phase_work(name, T, d_in, d_out, C, es):
    """(kind, amount): algorithmic FLOPs for GEMM phases, algorithmic HBM bytes for the
    fused elementwise passes (fwd reads h and writes h*m; bwd reads h and d(h*m) and
    writes dh; u is regenerated, never stored)."""
    table = {
        "transpose_inputs": ("byte", 2 * (T * d_in + d_in * C + C * d_out) * es),
        "gemm_target": ("flop", 2 * T * d_in * d_out),
        "gemm_xV": ("flop", 2 * T * d_in * C),
        "gate_mask_fwd": ("byte", 2 * T * C * es),
        "gemm_actsU": ("flop", 2 * T * C * d_out),
        "recon": ("byte", 3 * T * d_out * es),
        "loss_final": ("byte", 0),
        "gemm_dU": ("flop", 2 * T * C * d_out),
        "gemm_da": ("flop", 2 * T * C * d_out),
        "gate_mask_bwd": ("byte", 3 * T * C * es),
        "gate_grad_reduce": ("byte", 0),
        "gemm_dV": ("flop", 2 * T * d_in * C),
    }
    return table[name]


def cpu_baseline(T_sample, d_in, d_out, C, reps=3):
    import numpy as np

    from oracle import cpu
    from oracle import pd_oracle as po

    rng = np.random.default_rng(0)
    x = rng.normal(size=(T_sample, d_in)).astype(np.float32)
    W = (rng.normal(size=(d_out, d_in)) / np.sqrt(d_in)).astype(np.float32)
    V = (rng.normal(size=(d_in, C)) / np.sqrt(d_in)).astype(np.float32)
    U = (rng.normal(size=(C, d_out)) / np.sqrt(C)).astype(np.float32)
    gp = po.GateParams(rng.normal(size=(C, 16)).astype(np.float32) * 1.4, np.zeros((C, 16), np.float32),
                       rng.normal(size=(C, 16)).astype(np.float32) * 0.35, np.full(C, 0.3, np.float32))
    mk, dk = po.site_keys((0, 0), 0)
    cpu.dense_step(x, W, V, U, gp, mk, dk)  # warmup
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        cpu.dense_step(x, W, V, U, gp, mk, dk)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": T_sample / med, "unit": "tokens/s", "cores": cpu.num_threads(), "kind": "port",
            "sample": f"{T_sample} of the workload's tokens (same d_in/d_out/C), fp32 C+OpenMP restatement of the "
                      f"same step, median of {reps} after 1 warmup; {med * 1e3:.1f} ms per sample step"}


def rocprof_summary(db_path: str, command: str) -> str:
    """Per-kernel summary (calls, total/avg/min/max us, share) of a rocprofv3 results DB."""
    import sqlite3

    cur = sqlite3.connect(db_path).cursor()
    rows = list(cur.execute("select name, count(*), sum(duration), avg(duration), min(duration), max(duration) "
                            "from kernels group by name order by sum(duration) desc"))
    total = sum(r[2] for r in rows) or 1
    out = [f"command: `{command}`", "", "| kernel | calls | total us | avg us | min us | max us | % |",
           "|---|---|---|---|---|---|---|"]
    for name, n, tot, avg, mn, mx in rows:
        short = name.split("(")[0].replace("void ", "")
        out.append(f"| `{short}` | {n} | {tot / 1e3:.1f} | {avg / 1e3:.2f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} | "
                   f"{100 * tot / total:.1f} |")
    return "\n".join(out) + "\n"


def main():
    if "--rocprof-summary" in sys.argv:
        i = sys.argv.index("--rocprof-summary")
        db, cmd = sys.argv[i + 1], sys.argv[i + 2]
        print(rocprof_summary(db, cmd))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="dense768x3072_C4096", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-tokens", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every GPU box here has one MI355X; --gpus {args.gpus} is not run. "
              "Multi-GPU sharding is described in DESIGN.md, not measured.", file=sys.stderr)
        sys.exit(2)

    import torch

    from param_decomp_amd import hip_events
    from param_decomp_amd.dense_step import DenseSiteStep

    cfg = WORKLOADS[args.workload]
    T, d_in, d_out, C = cfg["T"], cfg["d_in"], cfg["d_out"], cfg["C"]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(T, d_in, device=dev, generator=gen).to(torch.bfloat16)
    W = (torch.randn(d_out, d_in, device=dev, generator=gen) / d_in**0.5).to(torch.bfloat16)
    V = (torch.randn(d_in, C, device=dev, generator=gen) / d_in**0.5).to(torch.bfloat16)
    U = (torch.randn(C, d_out, device=dev, generator=gen) / C**0.5).to(torch.bfloat16)
    gate = (torch.randn(C, 16, device=dev, generator=gen) * 2**0.5, torch.zeros(C, 16, device=dev),
            torch.randn(C, 16, device=dev, generator=gen) * (2 / 16) ** 0.5, torch.zeros(C, device=dev))
    step = DenseSiteStep(T, d_in, d_out, C, dtype=torch.bfloat16, device=dev, p=2.0, imp_coeff=1.0, recon_coeff=1.0)
    draw_key = (0, 0)
    from param_decomp_amd import prng

    def keys(i):
        return step.site_keys(prng.fold_in(draw_key, i), 0)

    for i in range(args.warmup):
        step.step(x, W, V, U, gate, *keys(i))
    nph = len(DenseSiteStep.PHASES)
    evs = [hip_events.create(nph + 1) for _ in range(args.steps)]
    arrs = [hip_events.array(e) for e in evs]
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hip_events.record(start, stream)
    for i in range(args.steps):
        step.step(x, W, V, U, gate, *keys(args.warmup + i), events=arrs[i])
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = hip_events.elapsed_ms(start, stop)
    ms_per_step = gpu_ms / args.steps
    phase_ms = {p: 0.0 for p in DenseSiteStep.PHASES}
    for e in evs:
        for j, p in enumerate(DenseSiteStep.PHASES):
            phase_ms[p] += hip_events.elapsed_ms(e[j], e[j + 1]) / args.steps
    for e in evs:
        hip_events.destroy(e)
    assert torch.isfinite(step.grads.losses).all(), step.grads.losses
    dom = max(phase_ms, key=phase_ms.get)
    kind, amount = phase_work(dom, T, d_in, d_out, C, 2)
    dur = phase_ms[dom] * 1e-3
    if kind == "flop":
        achieved = amount / dur / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_FLOPS / 1e12, "unit": "TFLOP/s",
                "frac": achieved / (PEAK_BF16_FLOPS / 1e12), "traffic": None, "kernel": dom,
                "avg_launch_ms": phase_ms[dom], "work_per_launch": amount}
    else:
        achieved = amount / dur / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": achieved / (PEAK_HBM / 1e9), "traffic": None, "kernel": dom,
                "avg_launch_ms": phase_ms[dom], "work_per_launch": amount}
    in_proj, out_proj = 2 * T * d_in * C, 2 * T * C * d_out
    step_flops = 2 * in_proj + 3 * out_proj  # reference rule: fwd in+out, bwd in + 2*out
    result = {
        "metric": METRIC,
        "value": T / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.randn of the named shapes; random-init U/V/gate)",
        "config": {"workload": args.workload, "tokens": T, "d_in": d_in, "d_out": d_out, "C": C, "gate_hidden": 16,
                   "imp_min": "p=2", "recon": "mse", "mask_draw": "threefry bf16 (partitionable)",
                   "parallelism": "single GPU"},
        "step_mfma_frac": step_flops / (ms_per_step * 1e-3) / PEAK_BF16_FLOPS,
        "step_tflops": step_flops / (ms_per_step * 1e-3) / 1e12,
        "wall_ms_per_step": wall * 1e3 / args.steps,
        "phases_ms": phase_ms,
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_tokens, d_in, d_out, C)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
