"""Masked-component fwd+bwd throughput on one MI355X.

Workloads (synthetic data of the named shapes, random-init weights):

- `qwen35moe4L` (default; the MoE stack the throughput target is quoted on): 4 layers of
  width 512, 42 experts with top-8 softmax routing, SwiGLU experts 512->256->512, every
  expert gate/up/down matrix decomposed with c=512 components per expert, 8192 tokens,
  bf16. A step is one `pd_moe_stack_step`: clean forward on the frozen experts, masked
  forward (grouped masked-component matmuls over bucketed tokens, with the frozen delta
  channel of the reference's stochastic masking), MSE recon of the final residual + L_p
  (p=2) imp-min over the selected CI, and the backward to every V/U and CI input.
- `llama4L`: the 4-layer Llama-style simple-MLP target (d_model 768, 12 heads, d_mlp
  3072, vocab 50277), every q/k/v/o (C=1024) and c_fc/down (C=4096) matrix decomposed,
  16 x 512 tokens, bf16. A step is one `pd_lm_stack_step`: frozen forward, masked
  forward with in-block mask and weight-delta draws, frozen causal attention, streamed
  KL over the tied head + L_p (p=2) imp-min, and the backward to every V/U and CI input.
- `dense768x3072_C4096`: one decomposed dense linear 768->3072, x bf16 [4096, 768],
  C=4096, per-component gate MLP hidden 16, bf16 Threefry mask uniforms, stochastic-
  recon MSE + sum_c mean_t |g_upper|^2 fwd+bwd (`pd_dense_step`).

Prints one JSON line: tokens/s, the roofline of the dominant kernel (its duration
measured with HIP events on the kernels' own stream inside the timed region), per-phase
times, and the CPU baseline (the oracle's restatement of the same step on a bounded
token sample, timed in this run on this host).

`python bench.py --rocprof-summary DB CMD` turns a rocprofv3 results DB into the
per-kernel table kept under profiles/ (no GPU needed).
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
PEAK_HBM = 8.0e12
METRIC = "masked-component fwd+bwd tokens/s on 1 MI355X; % of MFMA/HBM roofline"
DENSE = "dense768x3072_C4096"
MOE = "qwen35moe4L"
CI_MLP = "ci_mlp768_h1024_C4096"
CI_READOUT = "ci_readout_llama4L"
PPGD_DENSE = "ppgd_dense768x3072_C4096"
PPGD_MOE = "ppgd_qwen35moe4L"
PPGD_LLAMA = "ppgd_llama4L"
KL_STREAM = "kl_stream_llama4L"
FAITH_DENSE = "faith_dense768x3072_C4096"
FAITH_MOE = "faith_qwen35moe4L"
LLAMA = "llama4L"
TMS = "tms5_2"
RESID = "resid_mlp1L"
GEMM_MOE = "gemm_qwen35moe4L"
GEMM_LM = "gemm_llama4L"
PEAK_FP32_MFMA = 157.3e12
WORKLOADS = {
    DENSE: dict(T=4096, d_in=768, d_out=3072, C=4096),
    # with the frozen delta channel the reference's stochastic masking always draws
    MOE: dict(T=8192, d=512, f=256, E=42, k=8, c=512, L=4, use_delta=True),
    # the 4-layer Llama-style simple-MLP target: d_model 768, 12 heads (head_dim 64), d_mlp
    # 3072, vocab 50277, C = 1024 per attention matrix and 4096 per MLP matrix, 16 x 512
    # tokens, with the weight-delta channel of stochastic masking; KL over 3 vocab chunks
    LLAMA: dict(B=16, T=512, d=768, H=12, KV=12, f=3072, V=50277, L=4,
                C={"q_proj": 1024, "k_proj": 1024, "v_proj": 1024, "o_proj": 1024, "c_fc": 4096,
                   "down_proj": 4096}, n_chunks=3, use_delta=True),
    # the toy targets (fp32): TMS 5-2 (C=20, batch 4096, feature probability 0.05, p=1
    # imp-min) and ResidualMLP 1 layer (100 features in a 1000-d residual, MLP 1000->50->1000,
    # C=100 per matrix, batch 2048, probability 0.01, p=2 imp-min); per-component gate MLPs
    # hidden 16, stochastic recon MSE
    TMS: dict(B=4096, n_features=5, n_hidden=2, C=20, p_feat=0.05, low=0.0, p=1.0),
    RESID: dict(B=2048, n_features=100, d_embed=1000, d_mlp=50, C=100, p_feat=0.01, low=-1.0, p=2.0),
    CI_MLP: dict(T=4096, dims=(768, 1024, 4096)),
    # every q/k/v/o (C=768) and c_fc/down (C=3072) site of the 4-layer Llama-style target,
    # readouts side by side: 4 * (4*768 + 2*3072) components
    CI_READOUT: dict(T=8192, C=4 * (4 * 768 + 2 * 3072)),
    # streamed-vocab KL over the factored lm-head edge of the 4-layer Llama-style target:
    # 16 x 512 positions, d_model 768, vocab 50277 in 3 chunks (bf16)
    KL_STREAM: dict(N=16 * 512, d=768, V=50277, n_chunks=3),
    # persistent PGD on the dense site: per-token uint16 sources, momentum SGD, 2 warmup
    # ascents (the reference's LM PPGD setting)
    PPGD_DENSE: dict(T=4096, d_in=768, d_out=3072, C=4096, n_warmup=2, source_shape="bsc", source_dtype="uint16",
                     optimizer="momentum_sgd", momentum=0.9, lr=0.01),
    # persistent PGD over every expert site of the MoE stack: per-sample (bc) uint16 source
    # tables of 16 samples x 512 positions, momentum SGD, 2 warmup ascents
    PPGD_MOE: dict(T=8192, d=512, f=256, E=42, k=8, c=512, L=4, rows_per_source=512, n_warmup=2,
                   source_dtype="uint16", optimizer="momentum_sgd", momentum=0.9, lr=0.01),
    # persistent PGD over every decomposed matrix of the 4-layer Llama-style stack: one
    # source row per sample (bc: the reference's pooled adversary draws one particle per
    # sample), fp32 tables with the reference LM config's Adam (beta1 0.01, beta2 0.99,
    # lr 0.02), the delta leaf, 2 warmup ascents
    PPGD_LLAMA: dict(n_warmup=2, source_dtype="float32", optimizer="adam", beta1=0.01, beta2=0.99, lr=0.02),
    # faithfulness of the dense site, and of every expert matrix of the MoE stack (per kind:
    # 4 layers x 42 experts, each layer's experts one block-factored site)
    FAITH_DENSE: dict(groups=[dict(n=1, per=1, d_in=768, d_out=3072, C=4096)]),
    # the MoE step's grouped products in isolation (J = 8192 x 8 jobs over 42 experts with
    # ragged group sizes), each through the public grouped-GEMM entry points: the forward
    # products with the rhs K-contiguous (the step's per-step copies) and as stored
    # (MN-major), and the weight gradients from row-major (MN-major) and job-contiguous
    # (K-major) operands
    GEMM_MOE: dict(J=65536, E=42, d=512, f=256, c=512),
    # the LM step's dense products (16 x 512 tokens, d 768, d_mlp 3072, C 1024 / 4096, the
    # delta channel's concatenated contractions), C = A @ B^T with both operands
    # K-contiguous, each through pd_gemm and through torch.matmul (hipBLASLt) as a
    # library reference: (M, N, K, output dtype)
    GEMM_LM: dict(shapes=[(8192, 1024, 768, "bf16"), (8192, 4096, 768, "bf16"), (8192, 4096, 3072, "bf16"),
                          (8192, 768, 1792, "bf16"), (8192, 3072, 4864, "bf16"), (8192, 768, 7168, "bf16")]),
    FAITH_MOE: dict(groups=[dict(n=4 * 42, per=42, d_in=512, d_out=256, C=512),
                            dict(n=4 * 42, per=42, d_in=512, d_out=256, C=512),
                            dict(n=4 * 42, per=42, d_in=256, d_out=512, C=512)]),
}


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


def rocprof_csv_summary(stats_csv: str, command: str) -> str:
    """The per-kernel table of a rocprofv3 `--kernel-trace --stats` run's
    `*_kernel_stats.csv` (calls, total/avg/min/max us, share)."""
    import csv

    rows = list(csv.DictReader(open(stats_csv)))
    total = sum(float(r["TotalDurationNs"]) for r in rows) or 1.0
    out = [f"command: `{command}`", "", "| kernel | calls | total us | avg us | min us | max us | % |",
           "|---|---|---|---|---|---|---|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        short = r["Name"].split("(")[0].replace("void ", "")
        out.append(f"| `{short}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e3:.1f} | "
                   f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                   f"{float(r['MaxNs']) / 1e3:.2f} | {100 * float(r['TotalDurationNs']) / total:.1f} |")
    return "\n".join(out) + "\n"


def pmc_mfma_summary(csv1: str, csv2: str, command: str, n_xcd: int = 8, n_simd: int = 1024) -> str:
    """Per-kernel MFMA utilisation and instruction mix from two `--pmc` runs' counter
    CSVs: run 1 SQ_VALU_MFMA_BUSY_CYCLES, SQ_BUSY_CU_CYCLES, GRBM_GUI_ACTIVE; run 2
    SQ_INSTS_MFMA, SQ_INSTS_LDS, SQ_WAIT_INST_ANY, SQ_WAVE_CYCLES, SQ_INSTS_VALU.
    MFMA utilisation = MFMA busy cycles over (GPU-active cycles per XCD x SIMDs):
    GRBM_GUI_ACTIVE is summed over the 8 XCDs, and MI355X has 256 CUs x 4 SIMDs."""
    import collections
    import csv

    def load(path):
        per = collections.defaultdict(lambda: collections.defaultdict(float))
        name = {}
        for r in csv.DictReader(open(path)):
            d = int(r["Dispatch_Id"])
            per[d][r["Counter_Name"]] += float(r["Counter_Value"])
            per[d]["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            name[d] = r["Kernel_Name"].split("(")[0].replace("void ", "")
        agg = collections.defaultdict(lambda: collections.defaultdict(float))
        for d, v in per.items():
            for c, x in v.items():
                agg[name[d]][c] += x
            agg[name[d]]["calls"] += 1
        return agg

    a, b = load(csv1), load(csv2)
    out = [f"command: `{command}`", "",
           "| kernel | calls | avg us | MFMA util % | MFMA insts / call | LDS insts / MFMA | VALU insts / MFMA | "
           "wave cycles waiting % |", "|---|---|---|---|---|---|---|---|"]
    for n, v in sorted(a.items(), key=lambda kv: -kv[1]["ns"]):
        w = b.get(n, {})
        mf = w.get("SQ_INSTS_MFMA", 0.0)
        if not mf and not v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0):
            continue
        util = v["SQ_VALU_MFMA_BUSY_CYCLES"] / (v["GRBM_GUI_ACTIVE"] / n_xcd * n_simd) if v["GRBM_GUI_ACTIVE"] else 0
        calls = int(v["calls"])
        out.append(f"| `{n}` | {calls} | {v['ns'] / calls / 1e3:.1f} | {100 * util:.1f} | "
                   f"{mf / max(w.get('calls', 1), 1):.3g} | {w.get('SQ_INSTS_LDS', 0) / mf if mf else 0:.2f} | "
                   f"{w.get('SQ_INSTS_VALU', 0) / mf if mf else 0:.2f} | "
                   f"{100 * w.get('SQ_WAIT_INST_ANY', 0) / max(w.get('SQ_WAVE_CYCLES', 1), 1):.0f} |")
    return "\n".join(out) + "\n"


def copy_calibration():
    """Three device-to-device copies of 1 GiB (the plain copy kernel of known size that
    calibrates the FETCH_SIZE / WRITE_SIZE counters)."""
    import torch

    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print("copied", n)


RD_COUNTERS = ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum", "TCC_EA0_RDREQ_sum")


def pmc_traffic_summary(outdir: str, workloads) -> str:
    """HBM bytes per dispatch from two PMC runs per workload under OUTDIR: <name>_RD with the
    L2-to-memory read requests by size (bytes = 32 n32 + 64 n64 + 128 n128) and
    <name>_WRITE_SIZE; cal_* are the same runs around `bench.py --copy-calibration` (three
    1 GiB device copies), a check that the request-size sums give the bytes copied. The
    derived FETCH_SIZE counter is not used: it counts 128-byte reads through TCC_BUBBLE,
    which stays 0 on gfx950, so it reports half of every 128-byte read."""
    import collections
    import csv

    def load(path):
        """{label: {counter: [per-dispatch values]}}; a GEMM kernel (one template serves
        several phases) gets one row per grid size, labelled `name @work-items`."""
        agg = collections.defaultdict(lambda: collections.defaultdict(list))
        for r in csv.DictReader(open(os.path.join(outdir, path, "run_counter_collection.csv"))):
            k = r["Kernel_Name"].split("(")[0].replace("void ", "")
            if k.startswith("pd::k_gemm"):
                k = f"{k} @{r['Grid_Size']}"
            agg[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
        return agg

    def avg(d, c):
        v = d.get(c, [])
        return sum(v) / len(v) if v else 0.0

    def read_bytes(d):
        n32, n64, n128, n = (avg(d, c) for c in RD_COUNTERS)
        return 32 * n32 + 64 * n64 + 128 * n128, n - n32 - n64 - n128

    crd, cwr = load("cal_RD")["__amd_rocclr_copyBuffer"], load("cal_WRITE_SIZE")["__amd_rocclr_copyBuffer"]
    cal_rd, cal_unsized = read_bytes(crd)
    cal_wr = avg(cwr, "WRITE_SIZE") * 1024
    rd_cmd = "rocprofv3 --pmc " + " ".join(RD_COUNTERS)
    out = ["# HBM traffic per dispatch (rocprofv3 PMC)", "",
           "Two counter runs per workload: the L2-to-memory read requests by size (" + ", ".join(
               f"`{c}`" for c in RD_COUNTERS) + "; read bytes = 32 n32 + 64 n64 + 128 n128), then `WRITE_SIZE`.",
           "The derived `FETCH_SIZE` is not used: its formula counts 128-byte reads through `TCC_BUBBLE`, which",
           "stays 0 on gfx950, so it reports half of every 128-byte read.", "",
           "Check against three device-to-device copies of 1 GiB (`python3 bench.py --copy-calibration`):",
           f"read {cal_rd / 2**30:.4f} GiB and wrote {cal_wr / 2**30:.4f} GiB per copy "
           f"({cal_unsized:.0f} read requests of no listed size).", "",
           "commands (OUT = a fresh directory per run):", "", "```",
           f"cd /tmp && {rd_cmd} -d OUT -o run --output-format csv -- python3 bench.py --copy-calibration",
           "cd /tmp && rocprofv3 --pmc WRITE_SIZE -d OUT -o run --output-format csv -- python3 bench.py "
           "--copy-calibration"]
    for wl in workloads:
        out.append(f"cd /tmp && {rd_cmd} -d OUT -o run --output-format csv -- python3 bench.py "
                   f"--workload {wl} --steps 2 --warmup 1 --no-cpu-baseline")
        out.append(f"cd /tmp && rocprofv3 --pmc WRITE_SIZE -d OUT -o run --output-format csv -- python3 bench.py "
                   f"--workload {wl} --steps 2 --warmup 1 --no-cpu-baseline")
    out += ["```", f"summarized with `python bench.py --pmc-traffic-summary OUTDIR {' '.join(workloads)}`", ""]
    for wl in workloads:
        f, w = load(f"{wl}_RD"), load(f"{wl}_WRITE_SIZE")
        out += [f"## {wl}", "",
                "| kernel | dispatches | read MB/dispatch | 128-byte reads | write MB/dispatch | HBM bytes/dispatch |",
                "|---|---|---|---|---|---|"]
        rows = []
        for k in f:
            if k not in w or not k.startswith("pd::"):
                continue
            rb, _ = read_bytes(f[k])
            n128, n = avg(f[k], RD_COUNTERS[2]), avg(f[k], RD_COUNTERS[3])
            wb = avg(w[k], "WRITE_SIZE") * 1024
            nd = len(f[k][RD_COUNTERS[3]])
            rows.append(((rb + wb) * nd, k, nd, rb, n128 / max(n, 1), wb, rb + wb))
        for _, k, nd, rb, f128, wb, hbm in sorted(rows, reverse=True)[:24]:
            out.append(f"| `{k}` | {nd} | {rb / 1e6:.1f} | {100 * f128:.0f}% | {wb / 1e6:.1f} | {hbm:.4g} |")
        out.append("")
    return "\n".join(out) + "\n"


def pmc_l2_summary(csv_path: str, command: str, n_xcd: int = 8, n_ch: int = 16) -> str:
    """Per-kernel L2 behaviour from one `--pmc TCC_HIT_sum TCC_MISS_sum TCC_BUSY_sum
    TCC_EA0_RDREQ_sum GRBM_GUI_ACTIVE` run: hit rate, channel busy fraction (TCC_BUSY over
    GPU-active cycles per XCD x 16 channels per XCD) and memory read requests."""
    import collections
    import csv

    per = collections.defaultdict(lambda: collections.defaultdict(float))
    name = {}
    for r in csv.DictReader(open(csv_path)):
        dsp = int(r["Dispatch_Id"])
        per[dsp][r["Counter_Name"]] += float(r["Counter_Value"])
        per[dsp]["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        name[dsp] = r["Kernel_Name"].split("(")[0].replace("void ", "")
    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    for dsp, v in per.items():
        for c, x in v.items():
            agg[name[dsp]][c] += x
        agg[name[dsp]]["calls"] += 1
    out = [f"command: `{command}`", "", "| kernel | calls | avg us | L2 hit % | L2 channel busy % | memory read requests / call |",
           "|---|---|---|---|---|---|"]
    for n, v in sorted(agg.items(), key=lambda kv: -kv[1]["ns"]):
        if not n.startswith("pd::"):
            continue
        calls = int(v["calls"])
        hm = v["TCC_HIT_sum"] + v["TCC_MISS_sum"]
        busy = v["TCC_BUSY_sum"] / (v["GRBM_GUI_ACTIVE"] / n_xcd * n_xcd * n_ch) if v["GRBM_GUI_ACTIVE"] else 0
        out.append(f"| `{n}` | {calls} | {v['ns'] / calls / 1e3:.1f} | {100 * v['TCC_HIT_sum'] / hm if hm else 0:.1f} | "
                   f"{100 * busy:.0f} | {v['TCC_EA0_RDREQ_sum'] / calls:.3g} |")
    return "\n".join(out) + "\n"


# The kernel behind each phase, as named in profiles/hbm_traffic_pmc.md (a prefix of the
# demangled name: the phases of one kernel template share its per-dispatch average).
# Kernels of a timed phase (name prefixes as rocprofv3 prints them). A phase's traffic per
# launch is the dispatch-weighted mean over its kernels in the committed PMC summary.
PHASE_KERNEL = {
    # (the GEMM kernels of a phase also run in other phases: the clean pass, the backward)
    MOE: {"gemm_dw": ("pd::k_gemm_dtl<pd::DtlCfg<256, 256, 4, 2, 2, false>, float, 2,",
                      "pd::k_gemm_dtl<pd::DtlCfg<128, 128, 4, 2, 2, true>, float, 2,"),
          "gemm_fwd": ("pd::k_gemm_dtl<pd::DtlCfg<256, 256, 4, 2, 2, false>, unsigned short, 1, false, pd::EpiStore",
                       "pd::k_gemm_dtl<pd::DtlCfg<128, 128, 4, 2, 2, true>, unsigned short, 1, false, pd::EpiStore",
                       "pd::k_gemm_dtl_kcat<"),
          "gemm_dx": ("pd::k_gemm_dtl_kcat<",),
          "gemm_dx_mask": ("pd::k_gemm_dtl<pd::DtlCfg<256, 256, 4, 2, 2, false>, unsigned short, 1, false, "
                           "pd::EpiMaskBwd",
                           "pd::k_gemm_dtl<pd::DtlCfg<128, 128, 4, 2, 2, true>, unsigned short, 1, false, "
                           "pd::EpiMaskBwd"),
          "mask_fwd": ("pd::k_mask_fwd_tile",), "mask_bwd": ("pd::k_mask_bwd_tile", "pd::k_mask_bwd_vec")},
    # dense GEMM phases by template and grid (work-items: tiles x 512 threads at T 4096,
    # 768 -> 3072, C 4096; the 4096 x 4096 products run on 256x256 tiles)
    DENSE: {"gate_mask_fwd": ("pd::k_step_fwd_tab", "pd::k_gate_range", "pd::k_gate_table"),
            "gate_mask_bwd": ("pd::k_step_bwd",), "gate_grad_reduce": ("pd::k_gate_finalize",),
            "recon": ("pd::k_step_recon",),
            "gemm_target": ("pd::k_gemm_dtl<pd::DtlCfg<128, 128, 4, 2, 2, true>, unsigned short, 0, false, "
                            "pd::EpiStore, false, false> @393216",),
            "gemm_xV": ("pd::k_gemm_dtl<pd::DtlCfg<256, 256, 4, 2, 2, false>, unsigned short, 0, false, "
                        "pd::EpiStore, false, true> @131072",),
            "gemm_actsU": ("pd::k_gemm_dtl<pd::DtlCfg<128, 128, 4, 2, 2, true>, unsigned short, 0, false, "
                           "pd::EpiStore, false, true> @393216",),
            "gemm_dU": ("pd::k_gemm_dtl<pd::DtlCfg<128, 128, 4, 2, 2, true>, float, 0, false, "
                        "pd::EpiStore, true, true> @393216",),
            "gemm_da": ("pd::k_gemm_dtl<pd::DtlCfg<256, 256, 4, 2, 2, false>, unsigned short, 0, false, "
                        "pd::EpiStore, false, false> @131072",),
            "gemm_dV": ("pd::k_gemm_dtl<pd::DtlCfg<128, 128, 4, 2, 2, true>, float, 0, false, "
                        "pd::EpiStore, true, true> @98304",)},
}


def pmc_traffic(workload, phase):
    """HBM bytes per launch of the phase's kernels from the committed PMC summary (read
    requests by size plus WRITE_SIZE), or None."""
    prefixes = PHASE_KERNEL.get(workload, {}).get(phase)
    path = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")
    if prefixes is None or not os.path.exists(path):
        return None
    section, total, count = None, 0.0, 0
    for line in open(path):
        if line.startswith("## "):
            section = line[3:].strip()
        elif section == workload and line.startswith("| `") and line.split("`")[1].startswith(prefixes):
            cells = [c.strip() for c in line.rstrip().rstrip("|").split("|")]
            n = int(cells[2])
            total += float(cells[-1]) * n
            count += n
    return total / count if count else None


def roofline(kind, amount_per_launch, ms_per_launch, kernel, launches_per_step, traffic=None):
    dur = ms_per_launch * 1e-3
    if kind == "flop32":
        achieved = amount_per_launch / dur / 1e12
        return {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                "frac": achieved / (PEAK_FP32_MFMA / 1e12), "traffic": traffic, "kernel": kernel,
                "avg_launch_ms": ms_per_launch, "work_per_launch": amount_per_launch,
                "launches_per_step": launches_per_step, "precision": "fp32 MFMA (dense fp32 peak)"}
    if kind == "flop":
        achieved = amount_per_launch / dur / 1e12
        return {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_FLOPS / 1e12, "unit": "TFLOP/s",
                "frac": achieved / (PEAK_BF16_FLOPS / 1e12), "traffic": traffic, "kernel": kernel,
                "avg_launch_ms": ms_per_launch, "work_per_launch": amount_per_launch,
                "launches_per_step": launches_per_step}
    achieved = amount_per_launch / dur / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": achieved / (PEAK_HBM / 1e9), "traffic": traffic, "kernel": kernel, "avg_launch_ms": ms_per_launch,
            "work_per_launch": amount_per_launch, "launches_per_step": launches_per_step}


# ============================================================== dense single site
def dense_phase_work(name, T, d_in, d_out, C, es):
    """(kind, amount): algorithmic FLOPs for GEMM phases, algorithmic HBM bytes for the
    fused elementwise passes (fwd reads h and writes h*m; bwd reads h and d(h*m) and
    writes dh; u is regenerated or byte-stored, never stored at full width)."""
    table = {
        "delta_draw": ("byte", 4 * T),
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


def dense_cpu_baseline(T_sample, d_in, d_out, C, reps=20, warmup=3):
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
    for _ in range(warmup):
        cpu.dense_step(x, W, V, U, gp, mk, dk)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        cpu.dense_step(x, W, V, U, gp, mk, dk)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": T_sample / med, "unit": "tokens/s", "cores": cpu.num_threads(), "kind": "port",
            "sample": f"{T_sample} of the workload's tokens (same d_in/d_out/C), fp32 C+OpenMP restatement of the "
                      f"same step, median of {reps} after {warmup} warmups; {med * 1e3:.1f} ms per sample step"}


def run_dense(args):
    import torch

    from param_decomp_amd import hip_events, prng
    from param_decomp_amd.dense_step import DenseSiteStep

    cfg = WORKLOADS[DENSE]
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

    def keys(i):
        return step.site_keys(prng.fold_in((0, 0), i), 0)

    for i in range(args.warmup):
        step.step(x, W, V, U, gate, *keys(i))
    nph = len(DenseSiteStep.PHASES)
    evs = [hip_events.create(nph + 1) for _ in range(args.steps)]
    arrs = [hip_events.array(e) for e in evs]
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    torch.cuda.synchronize()
    hip_events.record(start, stream)
    for i in range(args.steps):
        step.step(x, W, V, U, gate, *keys(args.warmup + i), events=arrs[i])
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    ms_per_step = hip_events.elapsed_ms(start, stop) / args.steps
    phase_ms = {p: 0.0 for p in DenseSiteStep.PHASES}
    for e in evs:
        for j, p in enumerate(DenseSiteStep.PHASES):
            phase_ms[p] += hip_events.elapsed_ms(e[j], e[j + 1]) / args.steps
        hip_events.destroy(e)
    assert torch.isfinite(step.grads.losses).all(), step.grads.losses
    dom = max(phase_ms, key=phase_ms.get)
    kind, amount = dense_phase_work(dom, T, d_in, d_out, C, 2)
    in_proj, out_proj = 2 * T * d_in * C, 2 * T * C * d_out
    step_flops = 2 * in_proj + 3 * out_proj  # reference rule: fwd in+out, bwd in + 2*out (input not mask-dependent)
    res = {
        "tokens": T, "ms_per_step": ms_per_step,
        "config": {"workload": DENSE, "tokens": T, "d_in": d_in, "d_out": d_out, "C": C, "gate_hidden": 16,
                   "imp_min": "p=2", "recon": "mse", "mask_draw": "threefry bf16 (partitionable)"},
        "step_flops": step_flops, "phases_ms": phase_ms, "roofline": roofline(kind, amount, phase_ms[dom], dom, 1, pmc_traffic(DENSE, dom)),
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = dense_cpu_baseline(args.cpu_tokens, d_in, d_out, C)
    return res


# ============================================================== CI functions
def ci_cpu_baseline(workload, cfg, T_sample, reps=3):
    import numpy as np

    from oracle import ci_fn_oracle as co

    rng = np.random.default_rng(0)
    if workload == CI_MLP:
        weights, biases = co.init_mlp_stack(cfg["dims"], rng)
        x = rng.normal(size=(T_sample, cfg["dims"][0]))
        g = rng.normal(size=(T_sample, cfg["dims"][-1]))
        run = lambda: (co.site_mlp_fwd(x, weights, biases), co.site_mlp_bwd(x, weights, biases, g))
        what = f"SiteMLP {cfg['dims']} fwd+bwd"
    else:
        C = cfg["C"]
        h = rng.normal(size=(T_sample, C))
        params = np.stack([np.ones(C), np.zeros(C), np.ones(C), np.ones(C), np.zeros(C), np.ones(C), np.zeros(C)])
        g = rng.normal(size=(T_sample, C))
        run = lambda: (co.readout_fwd(h, params, h), co.readout_bwd(h, params, g))
        what = f"readout over {C} components fwd+bwd"
    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return {"value": T_sample / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{T_sample} tokens, NumPy float64 restatement of {what} (BLAS-threaded matmuls), median of "
                      f"{reps} after 1 warmup; {med * 1e3:.1f} ms per sample"}


def run_ci(args):
    """The engine's CI functions: a SiteMLP fwd+bwd (GEMMs with fused bias/GELU epilogues)
    or the component-activation readout fwd+bwd (one HBM-bound pass each way)."""
    import torch

    from param_decomp_amd import hip_events, ops

    cfg = WORKLOADS[args.workload]
    T = cfg["T"]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    stream = torch.cuda.current_stream().cuda_stream
    if args.workload == CI_MLP:
        dims = cfg["dims"]
        x = torch.randn(T, dims[0], device=dev, generator=gen).to(torch.bfloat16)
        ws = [(torch.randn(a, b, device=dev, generator=gen) * (2 / a) ** 0.5).to(torch.bfloat16)
              for a, b in zip(dims[:-1], dims[1:])]
        bs = [torch.zeros(b, device=dev, dtype=torch.bfloat16) for b in dims[1:]]
        g = torch.randn(T, dims[-1], device=dev, generator=gen).to(torch.bfloat16)
        fwd = lambda: ops.ci_mlp_fwd(x, ws, bs)
        bwd = lambda st: ops.ci_mlp_bwd(x, ws, g, st[1], False)
        mm = sum(2 * T * a * b for a, b in zip(dims[:-1], dims[1:]))
        work = {"fwd": ("flop", mm), "bwd": ("flop", 2 * mm - 2 * T * dims[0] * dims[1])}
        kernels = {"fwd": "ci_mlp_fwd (a bias+GELU-epilogue GEMM per layer, W^T copies)",
                   "bwd": "ci_mlp_bwd (dW GEMMs on K-contiguous copies, GELU'-epilogue d_a GEMMs, bias sums)"}
        config = {"workload": args.workload, "tokens": T, "dims": list(dims), "gelu": "erf", "d_x": False}
        step_flops = work["fwd"][1] + work["bwd"][1]
    else:
        C = cfg["C"]
        h = torch.randn(T, C, device=dev, generator=gen).to(torch.bfloat16)
        base = torch.randn(T, C, device=dev, generator=gen).to(torch.bfloat16)
        g = torch.randn(T, C, device=dev, generator=gen).to(torch.bfloat16)
        params = torch.stack([torch.rand(C, device=dev, generator=gen) + 0.5, torch.zeros(C, device=dev),
                              torch.ones(C, device=dev), torch.rand(C, device=dev, generator=gen) + 0.5,
                              torch.zeros(C, device=dev), torch.ones(C, device=dev), torch.zeros(C, device=dev)])
        fwd = lambda: ops.ci_readout_fwd(h, params, base)
        bwd = lambda st: ops.ci_readout_bwd(h, params, g)
        n = T * C
        work = {"fwd": ("byte", 6 * n), "bwd": ("byte", 6 * n)}  # fwd: h, base in, out; bwd: h, g in, d_h out
        kernels = {"fwd": "k_readout_fwd", "bwd": "k_readout_bwd (+ k_sum_parts)"}
        config = {"workload": args.workload, "tokens": T, "components": C, "base": True, "d_h": True}
        step_flops = 0
    for _ in range(args.warmup):
        bwd(fwd())
    evs = hip_events.create(3 * args.steps)
    torch.cuda.synchronize()
    for i in range(args.steps):
        hip_events.record(evs[3 * i], stream)
        st = fwd()
        hip_events.record(evs[3 * i + 1], stream)
        bwd(st)
        hip_events.record(evs[3 * i + 2], stream)
    torch.cuda.synchronize()
    phase = {"fwd": 0.0, "bwd": 0.0}
    for i in range(args.steps):
        phase["fwd"] += hip_events.elapsed_ms(evs[3 * i], evs[3 * i + 1]) / args.steps
        phase["bwd"] += hip_events.elapsed_ms(evs[3 * i + 1], evs[3 * i + 2]) / args.steps
    hip_events.destroy(evs)
    dom = max(phase, key=phase.get)
    kind, amount = work[dom]
    res = {"tokens": T, "ms_per_step": phase["fwd"] + phase["bwd"], "config": config, "step_flops": step_flops,
           "phases_ms": phase, "roofline": roofline(kind, amount, phase[dom], kernels[dom], 1,
                                                    pmc_traffic(args.workload, dom))}
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = ci_cpu_baseline(args.workload, cfg, args.cpu_tokens)
    return res


# ============================================================== streamed-vocab KL
def kl_cpu_baseline(cfg, N_sample, reps=3):
    import numpy as np

    from oracle import pd_oracle as po

    rng = np.random.default_rng(0)
    d, V = cfg["d"], cfg["V"]
    aq, ap = rng.normal(size=(N_sample, d)) * 0.5, rng.normal(size=(N_sample, d)) * 0.5
    hq, hp = rng.normal(size=(V, d)) * 0.05, rng.normal(size=(V, d)) * 0.05
    g = np.full(N_sample, 1.0 / N_sample)
    run = lambda: (po.streamed_position_kl(aq, hq, ap, hp, cfg["n_chunks"]),
                   po.streamed_position_kl_vjp(aq, hq, ap, hp, g))
    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return {"value": N_sample / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{N_sample} positions (full d and vocab), NumPy float64 restatement of the streamed KL and "
                      f"its input gradient (BLAS-threaded), median of {reps}; {med * 1e3:.1f} ms per sample"}


def run_kl(args):
    """Streamed-vocab KL fwd + bwd: per vocab chunk, the clean and masked logit blocks
    from the bf16 GEMM, the paired online-softmax update, and in the backward the
    re-derived logits' (q - p) g through the masked head."""
    import torch

    from param_decomp_amd import hip_events
    from param_decomp_amd.losses import streamed_position_kl

    cfg = WORKLOADS[args.workload]
    N, d, V, nc = cfg["N"], cfg["d"], cfg["V"], cfg["n_chunks"]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    aq = (torch.randn(N, d, device=dev, generator=gen) * 0.5).to(torch.bfloat16).requires_grad_(True)
    ap = (torch.randn(N, d, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    hq = (torch.randn(V, d, device=dev, generator=gen) * 0.05).to(torch.bfloat16)
    hp = (torch.randn(V, d, device=dev, generator=gen) * 0.05).to(torch.bfloat16)
    g = torch.full((N,), 1.0 / N, device=dev)
    for _ in range(args.warmup):
        torch.autograd.grad(streamed_position_kl(aq, hq, ap, hp, nc), aq, g)
    stream = torch.cuda.current_stream().cuda_stream
    evs = hip_events.create(3 * args.steps)
    torch.cuda.synchronize()
    for i in range(args.steps):
        hip_events.record(evs[3 * i], stream)
        kl = streamed_position_kl(aq, hq, ap, hp, nc)
        hip_events.record(evs[3 * i + 1], stream)
        torch.autograd.grad(kl, aq, g)
        hip_events.record(evs[3 * i + 2], stream)
    torch.cuda.synchronize()
    phase = {"fwd": 0.0, "bwd": 0.0}
    for i in range(args.steps):
        phase["fwd"] += hip_events.elapsed_ms(evs[3 * i], evs[3 * i + 1]) / args.steps
        phase["bwd"] += hip_events.elapsed_ms(evs[3 * i + 1], evs[3 * i + 2]) / args.steps
    hip_events.destroy(evs)
    assert torch.isfinite(kl).all()
    mm = 2 * N * d * V
    work = {"fwd": 2 * mm, "bwd": 3 * mm}
    dom = max(phase, key=phase.get)
    res = {"tokens": N, "ms_per_step": phase["fwd"] + phase["bwd"],
           "config": {"workload": args.workload, "positions": N, "d_model": d, "vocab": V, "n_vocab_chunks": nc},
           "step_flops": 5 * mm, "phases_ms": phase,
           "roofline": roofline("flop", work[dom], phase[dom],
                                {"fwd": "the chunk logit GEMMs (clean, masked) + k_kl_chunk",
                                 "bwd": "the re-derived chunk logits + k_kl_grad + the input-gradient GEMM"}[dom], 1)}
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = kl_cpu_baseline(cfg, args.cpu_tokens)
    return res


# ============================================================== persistent PGD
def ppgd_cpu_baseline(cfg, T_sample, reps=3):
    import numpy as np

    from oracle import pgd_oracle as po

    rng = np.random.default_rng(0)
    d_in, d_out, C = cfg["d_in"], cfg["d_out"], cfg["C"]
    x = rng.normal(size=(T_sample, d_in))
    V = rng.normal(size=(d_in, C)) / np.sqrt(d_in)
    U = rng.normal(size=(C, d_out)) / np.sqrt(C)
    ci = rng.uniform(size=(T_sample, C))
    tgt = rng.normal(size=(T_sample, d_out))
    src = rng.uniform(size=(T_sample, C))

    def run():
        s, vel = src.copy(), np.zeros_like(src)
        for it in range(cfg["n_warmup"] + 1):
            m = po.source_mask(ci, s, 1)
            xV = x @ V
            out = (xV * m) @ U
            g = 2 * (out - tgt) / out.size
            da = g @ U.T
            d_src, _ = po.source_mask_vjp(da * xV, ci, s, 1)
            if it == cfg["n_warmup"]:
                _ = (xV * m).T @ g, x.T @ (da * m)
            s, vel = po.momentum_sgd(s, d_src, vel, cfg["lr"], cfg["momentum"])

    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return {"value": T_sample / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{T_sample} tokens of the site (full widths), NumPy float64 restatement of the {cfg['n_warmup']} "
                      f"warmup ascents + final recon/backward/ascent (BLAS-threaded), median of {reps}; "
                      f"{med * 1e3:.1f} ms per sample step"}


def run_ppgd(args):
    """One persistent-PGD step of the dense site: n_warmup source ascents (masked forward,
    MSE, mask-only backward, source pullback, projected ascent) and the final forward and
    full backward with the final ascent."""
    import torch

    from param_decomp_amd import adversary as A
    from param_decomp_amd import hip_events, prng

    cfg = WORKLOADS[args.workload]
    T, d_in, d_out, C = cfg["T"], cfg["d_in"], cfg["d_out"], cfg["C"]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(T, d_in, device=dev, generator=gen).to(torch.bfloat16)
    V = (torch.randn(d_in, C, device=dev, generator=gen) / d_in**0.5).to(torch.bfloat16)
    U = (torch.randn(C, d_out, device=dev, generator=gen) / C**0.5).to(torch.bfloat16)
    ci = torch.rand(T, C, device=dev, generator=gen).to(torch.bfloat16)
    target = torch.randn(T, d_out, device=dev, generator=gen).to(torch.bfloat16)
    src = A.store_unit_float(torch.rand(T, C, device=dev, generator=gen), torch.uint16)
    adv = A.PersistentAdversary(src, A.MomentumSgdPGDConfig(cfg["momentum"]), cfg["n_warmup"], rows_per_source=1)
    step = A.DenseSitePPGDStep(adv)
    for i in range(args.warmup):
        step.step(x, V, U, ci, target, cfg["lr"], prng.fold_in((0, 0), i))
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    torch.cuda.synchronize()
    hip_events.record(start, stream)
    for i in range(args.steps):
        res = step.step(x, V, U, ci, target, cfg["lr"], prng.fold_in((0, 0), args.warmup + i))
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    ms = hip_events.elapsed_ms(start, stop) / args.steps
    hip_events.destroy([start, stop])
    assert torch.isfinite(res.loss).all()
    xv, uo = 2 * T * d_in * C, 2 * T * C * d_out
    warm = xv + 2 * uo          # fwd x@V, acts@U; bwd g@U^T only
    final = 2 * xv + 3 * uo     # fwd x@V, acts@U; bwd dU, da, dV
    step_flops = cfg["n_warmup"] * warm + final
    res_d = {"tokens": T, "ms_per_step": ms,
             "config": {"workload": args.workload, "tokens": T, "d_in": d_in, "d_out": d_out, "C": C,
                        "n_warmup": cfg["n_warmup"], "source_shape": cfg["source_shape"],
                        "source_dtype": cfg["source_dtype"], "optimizer": cfg["optimizer"],
                        "recon": "mse (site output)"},
             "step_flops": step_flops, "phases_ms": {"step": ms},
             "roofline": roofline("flop", step_flops, ms, "the step's bf16 GEMMs (x@V, acts@U, g@U^T; dU, dV "
                                  "in the final backward) with the source-mask and ascent passes", 1)}
    if not args.no_cpu_baseline:
        res_d["cpu_baseline"] = ppgd_cpu_baseline(cfg, args.cpu_tokens)
    return res_d


def run_ppgd_moe(args):
    """One persistent-PGD step over every expert site of the MoE stack: n_warmup
    source-only steps (masked forward, recon, backward to the sources, no weight
    gradients) each followed by a projected ascent of both source leaves, then the final
    step with every gradient and the final ascent."""
    import torch

    from param_decomp_amd import adversary as A
    from param_decomp_amd import hip_events, prng
    from param_decomp_amd.moe_step import MoEStackStep, MoEWeights

    cfg = WORKLOADS[PPGD_MOE]
    T, d, f, E, k, c, Ln = (cfg[x] for x in ("T", "d", "f", "E", "k", "c", "L"))
    rps = cfg["rows_per_source"]
    S = T // rps
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=dev, generator=g) * scale).to(torch.bfloat16)

    w = MoEWeights(ln=torch.zeros(Ln, d, device=dev), router=rn(Ln, E, d, scale=d**-0.5),
                   Wg=rn(Ln, E, d, f, scale=d**-0.5), Wu=rn(Ln, E, d, f, scale=d**-0.5),
                   Wd=rn(Ln, E, f, d, scale=f**-0.5), Vg=rn(Ln, E, d, c, scale=d**-0.5),
                   Ug=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vu=rn(Ln, E, d, c, scale=d**-0.5),
                   Uu=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vd=rn(Ln, E, f, c, scale=f**-0.5),
                   Ud=rn(Ln, E, c, d, scale=(E * c)**-0.5))
    x0 = rn(T, d, scale=1.0)
    ci = (torch.rand(Ln, 3, T, k, c, device=dev, generator=g) * 1.6 - 0.3).to(torch.bfloat16)
    step = MoEStackStep(T, d, f, E, k, c, Ln, device=dev, p=2.0, imp_coeff=0.0, recon_coeff=1.0, rows_per_source=rps)
    opt = A.MomentumSgdPGDConfig(cfg["momentum"])
    src = A.store_unit_float(torch.rand(Ln, 3, S, E, c, device=dev, generator=g), torch.uint16)
    srcd = A.store_unit_float(torch.rand(Ln, 3, S, device=dev, generator=g), torch.uint16)
    adv = A.PersistentAdversary(src, opt, cfg["n_warmup"], rows_per_source=rps)
    dadv = A.PersistentAdversary(srcd, opt, cfg["n_warmup"], rows_per_source=rps, leaf_index=1)
    ppgd = A.MoEPPGDStep(step, adv, dadv)
    for i in range(args.warmup):
        ppgd.step(x0, w, ci, cfg["lr"], prng.fold_in((0, 0), i))
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    torch.cuda.synchronize()
    hip_events.record(start, stream)
    for i in range(args.steps):
        res = ppgd.step(x0, w, ci, cfg["lr"], prng.fold_in((0, 0), args.warmup + i))
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    ms = hip_events.elapsed_ms(start, stop) / args.steps
    hip_events.destroy([start, stop])
    assert torch.isfinite(res.loss).all()
    gf = moe_gemm_flops(dict(cfg, use_delta=True))
    # a warmup step runs everything but the weight-gradient products
    step_flops = cfg["n_warmup"] * (sum(gf.values()) - gf["gemm_dw"]) + sum(gf.values())
    return {"tokens": T, "ms_per_step": ms,
            "config": {"workload": PPGD_MOE, "tokens": T, "width": d, "experts": E, "top_k": k, "expert_ffn": f,
                       "c_per_expert": c, "layers": Ln, "source_shape": "bc", "rows_per_source": rps,
                       "source_dtype": cfg["source_dtype"], "optimizer": cfg["optimizer"],
                       "n_warmup": cfg["n_warmup"], "recon": "mse(final residual)", "delta_source": True,
                       "mixers_and_shared_expert": "excluded"},
            "step_flops": step_flops, "phases_ms": {"step": ms},
            "roofline": roofline("flop", step_flops, ms, "the step's bf16 grouped GEMMs (warmup steps without "
                                 "the weight-gradient products) with the source-table mask passes and ascents", 1)}


def run_ppgd_llama(args):
    """One persistent-PGD step over every decomposed matrix of the LM stack (the llama4L
    shape): n_warmup source-only steps (masked forward, KL, backward to the sources, no
    weight gradients; the frozen forward formed once and reused) each followed by a
    projected ascent of every source leaf, then the final step with every gradient and the
    final ascent."""
    import torch

    from param_decomp_amd import adversary as A
    from param_decomp_amd import hip_events, prng
    from param_decomp_amd.lm_step import KINDS, LMStackStep, LMWeights

    lc, cfg = WORKLOADS[LLAMA], WORKLOADS[PPGD_LLAMA]
    B, T, d, H, KV, f, V, Ln = (lc[x] for x in ("B", "T", "d", "H", "KV", "f", "V", "L"))
    C, N = lc["C"], lc["B"] * lc["T"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=dev, generator=g) * scale).to(torch.bfloat16)

    dims = lm_site_dims(lc)
    w = LMWeights(wte=rn(V, d, scale=d**-0.5), ln1=torch.ones(Ln, d, device=dev), ln2=torch.ones(Ln, d, device=dev),
                  norm=torch.ones(d, device=dev),
                  W={k: rn(Ln, dims[k][1], dims[k][0], scale=dims[k][0]**-0.5) for k in KINDS},
                  V={k: rn(Ln, dims[k][0], C[k], scale=dims[k][0]**-0.5) for k in KINDS},
                  U={k: rn(Ln, C[k], dims[k][1], scale=C[k]**-0.5) for k in KINDS})
    ci = {k: (torch.rand(Ln, N, C[k], device=dev, generator=g) * 1.6 - 0.3).to(torch.bfloat16) for k in KINDS}
    tok = torch.randint(0, V, (N,), device=dev, generator=g, dtype=torch.int32)
    step = LMStackStep(B, T, d, H, KV, f, V, Ln, C, device=dev, p=2.0, imp_coeff=0.0, recon_coeff=1.0,
                       use_delta=True, n_kl_chunks=lc["n_chunks"], rows_per_source=T)
    opt = A.AdamPGDConfig(cfg["beta1"], cfg["beta2"])
    advs = {k: A.PersistentAdversary(torch.rand(Ln, B, C[k], device=dev, generator=g), opt, cfg["n_warmup"],
                                     rows_per_source=T, leaf_index=i) for i, k in enumerate(KINDS)}
    dadv = A.PersistentAdversary(torch.rand(Ln, len(KINDS), B, device=dev, generator=g), opt, cfg["n_warmup"],
                                 rows_per_source=T, leaf_index=len(KINDS))
    ppgd = A.LMPPGDStep(step, advs, dadv)
    for i in range(args.warmup):
        ppgd.step(tok, w, ci, cfg["lr"], prng.fold_in((0, 0), i))
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    torch.cuda.synchronize()
    hip_events.record(start, stream)
    for i in range(args.steps):
        res = ppgd.step(tok, w, ci, cfg["lr"], prng.fold_in((0, 0), args.warmup + i))
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    ms = hip_events.elapsed_ms(start, stop) / args.steps
    hip_events.destroy([start, stop])
    assert torch.isfinite(res.loss).all()
    gf = lm_gemm_flops(lc)
    # a warmup step runs everything but the weight-gradient products (and reuses the frozen forward)
    step_flops = cfg["n_warmup"] * (sum(gf.values()) - gf["gemm_dw"]) + sum(gf.values())
    return {"tokens": N, "ms_per_step": ms,
            "config": {"workload": PPGD_LLAMA, "batch": B, "seq_len": T, "d_model": d, "heads": H, "d_mlp": f,
                       "vocab": V, "layers": Ln, "C": dict(C), "source_shape": "bc", "rows_per_source": T,
                       "source_dtype": cfg["source_dtype"], "optimizer": cfg["optimizer"],
                       "n_warmup": cfg["n_warmup"], "recon": "kl(clean || masked), streamed over 3 vocab chunks",
                       "delta_source": True},
            "step_flops": step_flops, "phases_ms": {"step": ms},
            "roofline": roofline("flop", step_flops, ms, "the step's bf16 site, attention and KL GEMMs (warmup "
                                 "steps without the weight-gradient products) with the source-table mask passes "
                                 "and ascents", 1)}


# ============================================================== faithfulness
def faith_cpu_baseline(groups, reps=3):
    import numpy as np

    from oracle import faith_oracle as fo

    g0 = groups[0]
    n = min(g0["n"], 4)
    rng = np.random.default_rng(0)
    W = rng.normal(size=(n, g0["d_out"], g0["d_in"])).astype(np.float32)
    V = (rng.normal(size=(n, g0["d_in"], g0["C"])) / np.sqrt(g0["d_in"])).astype(np.float32)
    U = (rng.normal(size=(n, g0["C"], g0["d_out"])) / np.sqrt(g0["C"])).astype(np.float32)
    norms = (W.astype(np.float64) ** 2).reshape(n, -1).sum(1)
    run = lambda: (fo.site_errors(W, V, U, norms), fo.grads(W, V, U, norms, 1.0))
    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return {"value": n / med, "unit": "matrices/s", "cores": cores, "kind": "port",
            "sample": f"{n} matrices of the first group ({g0['d_out']}x{g0['d_in']}, C={g0['C']}), NumPy float64 "
                      f"restatement of loss + dV + dU (BLAS-threaded), median of {reps}; {med * 1e3:.1f} ms"}


def run_faith(args):
    """Faithfulness fwd+bwd over every group of the workload: fp32 MFMA products, the
    delta and its squared norm fused into the forward GEMM's epilogue."""
    import torch

    from param_decomp_amd import hip_events, ops

    groups = WORKLOADS[args.workload]["groups"]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    stacks = []
    for g in groups:
        W = torch.randn(g["n"], g["d_out"], g["d_in"], device=dev, generator=gen).to(torch.bfloat16)
        V = torch.randn(g["n"], g["d_in"], g["C"], device=dev, generator=gen) / g["d_in"] ** 0.5
        U = torch.randn(g["n"], g["C"], g["d_out"], device=dev, generator=gen) / g["C"] ** 0.5
        norms = (W.float() ** 2).reshape(g["n"] // g["per"], -1).sum(1)
        stacks.append((W, V, U, norms, g["per"]))
    n_sites = sum(g["n"] // g["per"] for g in groups)

    def fwd():
        return [ops.faithfulness_fwd(W, V, U, nt, per, 1.0 / n_sites, keep_delta=True) for W, V, U, nt, per in stacks]

    def bwd(outs):
        for (W, V, U, nt, per), (_, _, delta) in zip(stacks, outs):
            ops.faithfulness_bwd(delta, V, U, nt, per, 1.0 / n_sites, None)

    for _ in range(args.warmup):
        bwd(fwd())
    stream = torch.cuda.current_stream().cuda_stream
    evs = hip_events.create(3 * args.steps)
    torch.cuda.synchronize()
    for i in range(args.steps):
        hip_events.record(evs[3 * i], stream)
        outs = fwd()
        hip_events.record(evs[3 * i + 1], stream)
        bwd(outs)
        hip_events.record(evs[3 * i + 2], stream)
    torch.cuda.synchronize()
    phase = {"fwd": 0.0, "bwd": 0.0}
    for i in range(args.steps):
        phase["fwd"] += hip_events.elapsed_ms(evs[3 * i], evs[3 * i + 1]) / args.steps
        phase["bwd"] += hip_events.elapsed_ms(evs[3 * i + 1], evs[3 * i + 2]) / args.steps
    hip_events.destroy(evs)
    mm = sum(2 * g["n"] * g["d_in"] * g["d_out"] * g["C"] for g in groups)
    work = {"fwd": mm, "bwd": 2 * mm}
    dom = max(phase, key=phase.get)
    kern = {"fwd": "k_faith_gemm<EPI delta> (+ k_faith_reduce)", "bwd": "k_faith_gemm<EPI scale> x2 (dV, dU)"}[dom]
    n_mats = sum(g["n"] for g in groups)
    res = {"tokens": n_mats, "ms_per_step": phase["fwd"] + phase["bwd"],
           "config": {"workload": args.workload, "groups": groups, "W": "bf16", "V_U": "fp32 masters",
                      "unit_of_value": "matrices/s (a step is loss + dV + dU of every matrix)"},
           "step_flops": 3 * mm, "phases_ms": phase,
           "roofline": roofline("flop32", work[dom] / (len(groups) * (1 if dom == "fwd" else 2)),
                                phase[dom] / (len(groups) * (1 if dom == "fwd" else 2)), kern,
                                len(groups) * (1 if dom == "fwd" else 2))}
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = faith_cpu_baseline(groups)
    return res


def run_gemm_lm(args):
    """Each dense product of the LM step timed alone through pd_gemm, and the same product
    through torch.matmul (hipBLASLt) for reference; a step is one pd_gemm launch of every
    listed product. The two results are compared (max relative difference)."""
    import torch

    from param_decomp_amd import hip_events, ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    stream = torch.cuda.current_stream().cuda_stream
    reps = max(args.steps, 1)
    phase, tflops, lib_tflops, diff, flops = {}, {}, {}, {}, {}

    def timed(launch):
        for _ in range(max(args.warmup, 1)):
            launch()
        ev = hip_events.create(2)
        torch.cuda.synchronize()
        hip_events.record(ev[0], stream)
        for _ in range(reps):
            launch()
        hip_events.record(ev[1], stream)
        torch.cuda.synchronize()
        ms = hip_events.elapsed_ms(ev[0], ev[1]) / reps
        hip_events.destroy(ev)
        return ms

    for M, N, K, _ in WORKLOADS[GEMM_LM]["shapes"]:
        name = f"M{M}_N{N}_K{K}"
        a = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        b = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
        c_pd = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        c_lib = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        fl = 2 * M * N * K
        phase[name] = timed(lambda: ops.gemm(a, b, trans_b=True, out=c_pd))
        lib_ms = timed(lambda: torch.matmul(a, b.t(), out=c_lib))
        flops[name] = fl
        tflops[name] = fl / (phase[name] * 1e-3) / 1e12
        lib_tflops[name] = fl / (lib_ms * 1e-3) / 1e12
        diff[name] = float(((c_pd.float() - c_lib.float()).abs().max() / c_lib.float().abs().max()).item())
    dom = max(phase, key=phase.get)
    return {"tokens": 8192, "ms_per_step": sum(phase.values()),
            "config": {"workload": GEMM_LM, "shapes": WORKLOADS[GEMM_LM]["shapes"],
                       "unit_of_value": "token rows per step of every listed product"},
            "step_flops": sum(flops.values()), "phases_ms": phase, "tflops": tflops,
            "hipblaslt_tflops": lib_tflops, "max_rel_diff_vs_hipblaslt": diff,
            "roofline": roofline("flop", flops[dom], phase[dom], dom, 1)}


def run_gemm_moe(args):
    """Each grouped product of the MoE step timed alone (HIP events around the repeated
    launches of one product); a step is one launch of every listed product."""
    import torch

    from param_decomp_amd import hip_events, ops

    cfg = WORKLOADS[GEMM_MOE]
    J, E, d, f, c = cfg["J"], cfg["E"], cfg["d"], cfg["f"], cfg["c"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    w = torch.rand(E, generator=g, device=dev) * 0.8 + 0.6
    sizes = (w / w.sum() * J).floor().to(torch.int64)
    sizes[-1] += J - int(sizes.sum())
    offsets = torch.cat([torch.zeros(1, dtype=torch.int64, device=dev), sizes.cumsum(0)]).to(torch.int32)

    def rn(*shape):
        return torch.randn(*shape, device=dev, generator=g).to(torch.bfloat16)

    x, acts, din = rn(J, d), rn(J, c), rn(J, f)
    V, U, Vd = rn(E, d, c), rn(E, c, f), rn(E, f, c)
    Vt, Ut, Vdt = (t.transpose(1, 2).contiguous() for t in (V, U, Vd))
    dh, dg = rn(J, c), rn(J, f)
    xT, dhT, actsT, dgT = (t.t().contiguous() for t in (x, dh, acts, dg))
    prods = {  # name: (launch, FLOPs)
        "fwd_xV_K512_N512_rhsK": (lambda: ops.grouped_gemm(x, Vt, offsets, trans_rhs=True), 2 * J * d * c),
        "fwd_xV_K512_N512_rhsMN": (lambda: ops.grouped_gemm(x, V, offsets), 2 * J * d * c),
        "fwd_aU_K512_N256_rhsK": (lambda: ops.grouped_gemm(acts, Ut, offsets, trans_rhs=True), 2 * J * c * f),
        "fwd_aU_K512_N256_rhsMN": (lambda: ops.grouped_gemm(acts, U, offsets), 2 * J * c * f),
        "fwd_dinV_K256_N512_rhsK": (lambda: ops.grouped_gemm(din, Vdt, offsets, trans_rhs=True), 2 * J * f * c),
        "fwd_dinV_K256_N512_rhsMN": (lambda: ops.grouped_gemm(din, Vd, offsets), 2 * J * f * c),
        "dW_dV_512x512_MN": (lambda: ops.grouped_gemm_dw(x, dh, offsets, E, out_dtype=torch.float32), 2 * J * d * c),
        "dW_dV_512x512_K": (lambda: ops.grouped_gemm_dw_kmajor(xT, dhT, offsets, E, out_dtype=torch.float32),
                            2 * J * d * c),
        "dW_dU_512x256_MN": (lambda: ops.grouped_gemm_dw(acts, dg, offsets, E, out_dtype=torch.float32),
                             2 * J * c * f),
        "dW_dU_512x256_K": (lambda: ops.grouped_gemm_dw_kmajor(actsT, dgT, offsets, E, out_dtype=torch.float32),
                            2 * J * c * f),
    }
    stream = torch.cuda.current_stream().cuda_stream
    reps = max(args.steps, 1)
    phase, tflops = {}, {}
    for name, (launch, fl) in prods.items():
        for _ in range(max(args.warmup, 1)):
            launch()
        ev = hip_events.create(2)
        torch.cuda.synchronize()
        hip_events.record(ev[0], stream)
        for _ in range(reps):
            launch()
        hip_events.record(ev[1], stream)
        torch.cuda.synchronize()
        phase[name] = hip_events.elapsed_ms(ev[0], ev[1]) / reps
        hip_events.destroy(ev)
        tflops[name] = fl / (phase[name] * 1e-3) / 1e12
    # The bar: the dense equivalents (all J rows against one weight) through hipBLASLt
    # (torch.matmul) and through pd_gemm; not part of the step.
    dense_bar = {}
    for M, K, N in ((J, d, c), (J, c, f), (J, f, c)):
        a = rn(M, K)
        bt = rn(N, K)
        out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        times = {}
        for lib, launch in (("hipblaslt", lambda: torch.matmul(a, bt.t(), out=out)),
                            ("pd_gemm", lambda: ops.gemm(a, bt, trans_b=True, out=out))):
            for _ in range(max(args.warmup, 1)):
                launch()
            ev = hip_events.create(2)
            torch.cuda.synchronize()
            hip_events.record(ev[0], stream)
            for _ in range(reps):
                launch()
            hip_events.record(ev[1], stream)
            torch.cuda.synchronize()
            times[lib] = hip_events.elapsed_ms(ev[0], ev[1]) / reps
            hip_events.destroy(ev)
        dense_bar[f"M{M}_K{K}_N{N}"] = {lib: {"ms": t, "tflops": 2 * M * N * K / (t * 1e-3) / 1e12}
                                        for lib, t in times.items()}
    dom = max(phase, key=phase.get)
    return {"tokens": J, "ms_per_step": sum(phase.values()),
            "config": {"workload": GEMM_MOE, **cfg, "group_sizes": "ragged, seeded (0.6 + 0.8 U) weights",
                       "unit_of_value": "job rows per step of every listed product"},
            "step_flops": sum(fl for _, fl in prods.values()), "phases_ms": phase, "tflops": tflops,
            "dense_equivalents": dense_bar,
            "roofline": roofline("flop", prods[dom][1], phase[dom], dom, 1)}


# ============================================================== MoE stack
def moe_site_flops(J, d, f, c):
    """Per-site (in_proj, out_proj) FLOPs: gate/up read width d and write f; down reads
    f and writes d (reference rule, `pd/core/flops/target.py:39-93`)."""
    return {"gate": (2 * J * d * c, 2 * J * c * f), "up": (2 * J * d * c, 2 * J * c * f),
            "down": (2 * J * f * c, 2 * J * c * d)}


def moe_gemm_flops(cfg):
    """Per-category GEMM FLOPs of one step by the reference's linear rule
    (`pd/core/flops/target.py:53-93`): a decomposed site costs in_proj + out_proj forward
    (+ the frozen product W when the delta channel is on), and in backward in_proj per
    gradient formed (input, components), out_proj twice (mask, components) and the frozen
    product once more for the input gradient. Layer 0's gate/up inputs carry no mask
    dependence: no input gradient there, and their frozen products are the clean pass's
    (shared)."""
    J, d, f, c, E, T = cfg["T"] * cfg["k"], cfg["d"], cfg["f"], cfg["c"], cfg["E"], cfg["T"]
    per = moe_site_flops(J, d, f, c)
    frozen = 2 * J * d * f if cfg.get("use_delta", True) else 0
    fwd = dx = dw = 0
    for layer in range(cfg["L"]):
        for s, (i, o) in per.items():
            changed = not (layer == 0 and s != "down")
            fwd += i + o + frozen * changed
            dx += o + (i + frozen) * changed
            dw += i + o
    clean = cfg["L"] * (2 * T * d * E + 3 * 2 * J * d * f)  # the clean pass's router and expert products
    router = (cfg["L"] - 1) * 2 * (2 * T * d * E)  # masked-pass router fwd + input grad, layers >= 1
    return {"gemm_fwd": fwd, "gemm_dx": dx, "gemm_dw": dw, "clean": clean, "router": router}


def moe_step_flops(cfg):
    return sum(moe_gemm_flops(cfg).values())


def moe_dacts_work(cfg):
    """The d_acts products (g @ U^T per site and layer; part of gemm_dx's FLOPs) that run
    with the mask backward as their epilogue: their FLOPs and algorithmic HBM bytes (read
    g [J, K] and U; the epilogue reads ci, h, the u byte and writes d_h, d_ci: 9 bytes per
    selected component)."""
    J, d, f, c, E = cfg["T"] * cfg["k"], cfg["d"], cfg["f"], cfg["c"], cfg["E"]
    flops = byts = 0
    for _ in range(cfg["L"]):
        for K in (f, f, d):  # gate, up (g has width f), down (width d)
            flops += 2 * J * c * K
            byts += 2 * J * K + 2 * E * K * c + 9 * J * c
    return flops, byts


def moe_cpu_baseline(cfg, T_sample, reps=20, warmup=3):
    """The compiled fp32 C/OpenMP restatement of the same step (`oracle/cpu_step.c`
    `or_moe_step`, checked against the NumPy oracle) on `T_sample` tokens at the full
    widths; inputs packed once outside the timed calls."""
    import numpy as np

    from oracle import cpu
    from oracle import moe_oracle as mo

    mc = mo.MoEConfig(T=T_sample, d=cfg["d"], f=cfg["f"], E=cfg["E"], k=cfg["k"], c=cfg["c"], L=cfg["L"])
    params, x0, ci = mo.init_moe(mc, np.random.default_rng(0))
    st = cpu.pack_moe(mc, params, x0, ci, (0, 1))
    for _ in range(warmup):
        cpu.run_moe(mc, st, use_delta=cfg["use_delta"])
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        cpu.run_moe(mc, st, use_delta=cfg["use_delta"])
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": T_sample / med, "unit": "tokens/s", "cores": cpu.num_threads(), "kind": "port",
            "sample": f"{T_sample} of the workload's 8192 tokens (full widths, 42 experts, 4 layers), the fp32 "
                      f"C/OpenMP restatement of the same step (oracle/cpu_step.c), median of {reps} after {warmup} "
                      f"warmups; {med * 1e3:.0f} ms per sample step"}


def run_moe(args):
    import torch

    from param_decomp_amd import hip_events, prng
    from param_decomp_amd.moe_step import CATEGORIES, MoEStackStep, MoEWeights

    cfg = WORKLOADS[MOE]
    T, d, f, E, k, c, Ln = (cfg[x] for x in ("T", "d", "f", "E", "k", "c", "L"))
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=dev, generator=g) * scale).to(torch.bfloat16)

    # V by its per-block fan-in, U by the site's C = E*c (the reference's blocked init,
    # BLOCKED_U_INIT_FAN_IN = "site", pd/core/components.py:639-677)
    w = MoEWeights(ln=torch.zeros(Ln, d, device=dev), router=rn(Ln, E, d, scale=d**-0.5),
                   Wg=rn(Ln, E, d, f, scale=d**-0.5), Wu=rn(Ln, E, d, f, scale=d**-0.5),
                   Wd=rn(Ln, E, f, d, scale=f**-0.5), Vg=rn(Ln, E, d, c, scale=d**-0.5),
                   Ug=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vu=rn(Ln, E, d, c, scale=d**-0.5),
                   Uu=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vd=rn(Ln, E, f, c, scale=f**-0.5),
                   Ud=rn(Ln, E, c, d, scale=(E * c)**-0.5))
    x0 = rn(T, d, scale=1.0)
    ci = (torch.rand(Ln, 3, T, k, c, device=dev, generator=g) * 1.6 - 0.3).to(torch.bfloat16)
    step = MoEStackStep(T, d, f, E, k, c, Ln, device=dev, p=2.0, imp_coeff=1.0, recon_coeff=1.0,
                        use_delta=cfg["use_delta"])
    for i in range(args.warmup):
        step.step(x0, w, ci, prng.fold_in((0, 0), i))
    cap = 1024
    evs = [hip_events.create(cap) for _ in range(args.steps)]
    arrs = [hip_events.array(e) for e in evs]
    cats = [torch.zeros(cap, dtype=torch.int32) for _ in range(args.steps)]
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    counts = []
    torch.cuda.synchronize()
    hip_events.record(start, stream)
    for i in range(args.steps):
        counts.append(step.step_timed(x0, w, ci, prng.fold_in((0, 0), args.warmup + i), arrs[i], cats[i]))
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    ms_per_step = hip_events.elapsed_ms(start, stop) / args.steps
    cat_ms = {name: 0.0 for name in CATEGORIES}
    cat_n = {name: 0 for name in CATEGORIES}
    for e, cc, n in zip(evs, cats, counts):
        for j in range(n - 1):
            name = CATEGORIES[int(cc[j])]
            cat_ms[name] += hip_events.elapsed_ms(e[j], e[j + 1]) / args.steps
            cat_n[name] += 1
        hip_events.destroy(e)
    for name in cat_n:
        cat_n[name] //= args.steps
    assert torch.isfinite(step.losses).all(), step.losses
    # algorithmic work per category (per step) for the roofline of the dominant one
    J = T * k
    gf = moe_gemm_flops(cfg)
    da_flops, da_bytes = moe_dacts_work(cfg)
    fused = cat_n.get("gemm_dx_mask", 0) > 0  # the d_acts products carry the mask backward
    work = {
        "gemm_fwd": ("flop", gf["gemm_fwd"]),
        "gemm_dx": ("flop", gf["gemm_dx"] - (da_flops if fused else 0)),
        "gemm_dw": ("flop", gf["gemm_dw"]),
        "mask_fwd": ("byte", Ln * 3 * J * c * (2 + 2 + 2 + 1)),   # read ci, h; write acts, u bits
        "gemm_dx_mask": ("byte", da_bytes),  # HBM-bound: 9 B per element against ~2 flop/B
    }
    if not fused:
        work["mask_bwd"] = ("byte", Ln * 3 * J * c * (2 + 2 + 1 + 2 + 2))  # read ci, h, u, d_acts; write d_h, d_ci
    dom = max((n for n in cat_ms if n in work), key=cat_ms.get)
    kind, amount = work[dom]
    launches = cat_n[dom]
    roof = roofline(kind, amount / launches, cat_ms[dom] / launches, dom, launches, pmc_traffic(MOE, dom))
    res = {
        "tokens": T, "ms_per_step": ms_per_step,
        "config": {"workload": MOE, "tokens": T, "width": d, "experts": E, "top_k": k, "expert_ffn": f,
                   "c_per_expert": c, "layers": Ln, "imp_min": "p=2", "recon": "mse(final residual)",
                   "mask_draw": "threefry bf16 (partitionable)", "delta_channel": cfg["use_delta"],
                   "mixers_and_shared_expert": "excluded"},
        "step_flops": moe_step_flops(cfg), "phases_ms": cat_ms, "launches_per_step": cat_n, "roofline": roof,
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = moe_cpu_baseline(cfg, args.cpu_tokens)
    return res


# ============================================================== toy targets
def toy_flops(workload, cfg):
    """Reference rule per site (`pd/core/flops/target.py:39-93`): forward in + out, backward
    in (component gradient; the toys' first site reads the data) or 2 in (later sites)
    + 2 out, plus the per-component gate MLP's 2 * 2 * 16 multiply-adds per (row, component)
    forward and twice that backward (elementwise by the rule, counted here as work)."""
    B = cfg["B"]
    if workload == TMS:
        sites = [(cfg["n_features"], cfg["n_hidden"], False), (cfg["n_hidden"], cfg["n_features"], True)]
    else:
        sites = [(cfg["d_embed"], cfg["d_mlp"], False), (cfg["d_mlp"], cfg["d_embed"], True)]
    total = 0
    for din, dout, dx in sites:
        i, o = 2 * B * din * cfg["C"], 2 * B * cfg["C"] * dout
        total += (i + o) + (i * (1 + dx) + 2 * o)
    return total


def toy_cpu_baseline(workload, cfg, reps=5):
    import numpy as np

    from oracle import toy_oracle as to

    rng = np.random.default_rng(0)
    if workload == TMS:
        tc = to.TMSConfig(n_features=cfg["n_features"], n_hidden=cfg["n_hidden"], C=cfg["C"], batch=cfg["B"])
        target, sites = to.tms_init(tc, rng)
        x = to.tms_batch(tc, rng)
        kind = "tms"
    else:
        rc = to.ResidMLPConfig(n_features=cfg["n_features"], d_embed=cfg["d_embed"], d_mlp=cfg["d_mlp"], n_layers=1,
                               C=cfg["C"], batch=cfg["B"])
        target, sites = to.resid_mlp_init(rc, rng)
        x = to.resid_mlp_batch(rc, rng)
        kind = "resid_mlp"
    run = lambda: to.toy_step(kind, target, sites, x, (0, 1), p=cfg["p"])
    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return {"value": cfg["B"] / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"the whole {cfg['B']}-row batch, the toy oracle's NumPy float64 restatement of the same step "
                      f"(BLAS-threaded matmuls), median of {reps} after 1 warmup; {med * 1e3:.2f} ms per step"}


def run_toy(args):
    """The toy decomposition step: clean forward, per-site gate MLPs and CI, Threefry
    masks (fp32 draws), masked forward, MSE + L_p imp-min and the backward. TMS runs as one
    fused kernel (pd_tms_step); ResidMLP as one native call (pd_resid_mlp_step: the fp32
    products and one fused CI / mask pass per site and direction)."""
    import torch

    from param_decomp_amd import hip_events, prng, toys

    cfg = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    if args.workload == TMS:
        target, sites = toys.init_tms(cfg["n_features"], cfg["n_hidden"], cfg["C"], device=dev, generator=g)
    else:
        target, sites = toys.init_resid_mlp(cfg["n_features"], cfg["d_embed"], cfg["d_mlp"], 1, cfg["C"],
                                            device=dev, generator=g)
    x = toys.sparse_features(cfg["B"], cfg["n_features"], cfg["p_feat"], cfg["low"], device=dev, generator=g)
    if args.workload == TMS:  # one fused launch (+ one reduction) per step
        step = toys.TMSFusedStep(target, sites, p=cfg["p"], imp_coeff=1.0, recon_coeff=1.0)
    else:  # one native call per step
        step = toys.ResidMLPFusedStep(target, sites, p=cfg["p"], imp_coeff=1.0, recon_coeff=1.0)
    for i in range(args.warmup):
        step.step(x, prng.fold_in((0, 0), i))
    keys = [prng.fold_in((0, 0), args.warmup + i) for i in range(args.steps)]  # the training loop's step keys
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    torch.cuda.synchronize()
    hip_events.record(start, stream)
    for i in range(args.steps):
        res = step.step(x, keys[i])
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    ms = hip_events.elapsed_ms(start, stop) / args.steps
    hip_events.destroy([start, stop])
    assert torch.isfinite(res["loss"]).all()
    flops = toy_flops(args.workload, cfg)
    out = {"tokens": cfg["B"], "ms_per_step": ms,
           "config": {"workload": args.workload, **{k: v for k, v in cfg.items()}, "dtype": "fp32",
                      "gate_hidden": 16, "recon": "mse", "mask_draw": "threefry fp32 (partitionable)"},
           "step_flops": flops, "phases_ms": {"step": ms},
           "roofline": dict(roofline("flop32", flops, ms, "whole step" if args.workload == TMS else
                                     "whole step (fp32, one native call of 31 launches)", 1),
                            note="TMS: one fused launch (k_tms_step) plus one reduction per step, bound by the "
                                 "CI gates' exact-erf GELUs and the Threefry draws on the vector ALUs; the FLOPs "
                                 "counted (the reference rule) are only its tiny contractions" if args.workload == TMS
                            else "one native call (pd_resid_mlp_step): 17 fp32 GEMMs of 2048 rows over d "
                                 "1000/100/50, one fused CI / mask pass per site forward and backward, relu, recon "
                                 "and loss passes; its contractions are microseconds of fp32 MFMA work each")}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = toy_cpu_baseline(args.workload, cfg)
    return out


# ============================================================== Llama-style LM stack
def lm_site_dims(cfg):
    qd, kvd = cfg["H"] * 64, cfg["KV"] * 64
    d, f = cfg["d"], cfg["f"]
    return {"q_proj": (d, qd), "k_proj": (d, kvd), "v_proj": (d, kvd), "o_proj": (qd, d), "c_fc": (d, f),
            "down_proj": (f, d)}


def lm_gemm_flops(cfg):
    """Per-category FLOPs of one step by the reference's linear rule
    (`pd/core/flops/target.py:39-93`, frozen paths included with the weight-delta channel):
    forward in + out (+ frozen); backward in * (input grad + component grad) + out * 2
    (+ frozen for the input gradient). Layer 0's q/k/v read the embedding: no input
    gradient there. Attention is a frozen product pair, full T x T per head, forward and
    backward."""
    N = cfg["B"] * cfg["T"]
    fwd = dx = dw = 0
    frozen_on = cfg.get("use_delta", True)
    for layer in range(cfg["L"]):
        for k, (din, dout) in lm_site_dims(cfg).items():
            C = cfg["C"][k]
            i, o, fr = 2 * N * din * C, 2 * N * C * dout, 2 * N * din * dout * frozen_on
            ig = not (layer == 0 and k in ("q_proj", "k_proj", "v_proj"))
            fwd += i + o + fr
            dx += o + (i + fr) * ig
            dw += i + o
    attn_one = 2 * cfg["B"] * cfg["H"] * cfg["T"] * cfg["T"] * 64  # one T x T x 64 product over all heads
    clean = sum(2 * N * din * dout for din, dout in lm_site_dims(cfg).values()) * cfg["L"] + 2 * attn_one * cfg["L"]
    kl = 2 * N * cfg["d"] * cfg["V"] * 5  # fwd: clean + masked logits; bwd: both again + the input gradient
    return {"gemm_fwd": fwd, "gemm_dx": dx, "gemm_dw": dw, "attention": 6 * attn_one * cfg["L"], "clean": clean,
            "kl": kl}


def lm_cpu_baseline(cfg, n_sample, reps=20, warmup=3):
    """The LM oracle's step in fp32 (torch on the host cores) on `n_sample` tokens of one
    sequence at the workload's full widths."""
    import numpy as np
    import torch

    from oracle import lm_oracle as lo

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    torch.set_num_threads(cores)
    lc = lo.LMConfig(n_layers=cfg["L"], d=cfg["d"], n_head=cfg["H"], n_kv_head=cfg["KV"], d_mlp=cfg["f"],
                     vocab=cfg["V"], C=dict(cfg["C"]))
    rng = np.random.default_rng(0)
    params = lo.init_lm(lc, rng)
    tokens = rng.integers(0, lc.vocab, size=(1, n_sample))
    ci = lo.init_ci(lc, n_sample, rng)
    run = lambda: lo.lm_stack_step(lc, params, tokens, ci, (0, 1), use_delta=cfg["use_delta"], dtype=torch.float32)
    for _ in range(warmup):
        run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": n_sample / med, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"one sequence of {n_sample} tokens at the full widths (4 layers, vocab 50277), the oracle's "
                      f"torch fp32 CPU restatement of the same step (autograd backward), median of {reps} after "
                      f"{warmup} warmups; {med * 1e3:.0f} ms per sample step"}


def run_llama(args):
    import torch

    from param_decomp_amd import hip_events, prng
    from param_decomp_amd.lm_step import CATEGORIES, KINDS, LMStackStep, LMWeights

    cfg = WORKLOADS[LLAMA]
    B, T, d, H, KV, f, V, Ln = (cfg[x] for x in ("B", "T", "d", "H", "KV", "f", "V", "L"))
    C = cfg["C"]
    N = B * T
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=dev, generator=g) * scale).to(torch.bfloat16)

    dims = lm_site_dims(cfg)
    # target N(0, d_in^-1/2); components V by d_in^-1/2, U by C^-1/2 (pd/core/components.py:650-677)
    w = LMWeights(wte=rn(V, d, scale=d**-0.5), ln1=torch.ones(Ln, d, device=dev), ln2=torch.ones(Ln, d, device=dev),
                  norm=torch.ones(d, device=dev),
                  W={k: rn(Ln, dims[k][1], dims[k][0], scale=dims[k][0]**-0.5) for k in KINDS},
                  V={k: rn(Ln, dims[k][0], C[k], scale=dims[k][0]**-0.5) for k in KINDS},
                  U={k: rn(Ln, C[k], dims[k][1], scale=C[k]**-0.5) for k in KINDS})
    ci = {k: (torch.rand(Ln, N, C[k], device=dev, generator=g) * 1.6 - 0.3).to(torch.bfloat16) for k in KINDS}
    tok = torch.randint(0, V, (N,), device=dev, generator=g, dtype=torch.int32)
    step = LMStackStep(B, T, d, H, KV, f, V, Ln, C, device=dev, p=2.0, imp_coeff=1.0, recon_coeff=1.0,
                       use_delta=cfg["use_delta"], n_kl_chunks=cfg["n_chunks"])
    for i in range(args.warmup):
        step.step(tok, w, ci, prng.fold_in((0, 0), i))
    cap = 2048
    evs = [hip_events.create(cap) for _ in range(args.steps)]
    arrs = [hip_events.array(e) for e in evs]
    cats = [torch.zeros(cap, dtype=torch.int32) for _ in range(args.steps)]
    stream = torch.cuda.current_stream().cuda_stream
    start, stop = hip_events.create(2)
    counts = []
    torch.cuda.synchronize()
    hip_events.record(start, stream)
    for i in range(args.steps):
        counts.append(step.step_timed(tok, w, ci, prng.fold_in((0, 0), args.warmup + i), arrs[i], cats[i]))
    hip_events.record(stop, stream)
    torch.cuda.synchronize()
    ms_per_step = hip_events.elapsed_ms(start, stop) / args.steps
    cat_ms = {name: 0.0 for name in CATEGORIES}
    cat_n = {name: 0 for name in CATEGORIES}
    for e, cc, n in zip(evs, cats, counts):
        for j in range(n - 1):
            name = CATEGORIES[int(cc[j])]
            cat_ms[name] += hip_events.elapsed_ms(e[j], e[j + 1]) / args.steps
            cat_n[name] += 1
        hip_events.destroy(e)
    for name in cat_n:
        cat_n[name] //= args.steps
    assert torch.isfinite(step.losses).all(), step.losses
    gf = lm_gemm_flops(cfg)
    sumC = sum(C[k] for k in KINDS) * Ln
    work = {
        "gemm_fwd": ("flop", gf["gemm_fwd"]),
        "gemm_dx": ("flop", gf["gemm_dx"]),
        "gemm_dw": ("flop", gf["gemm_dw"]),
        "mask_fwd": ("byte", N * sumC * (2 + 2 + 2 + 1)),   # read ci, xV; write acts, u bits
        "mask_bwd": ("byte", N * sumC * (2 + 2 + 1 + 2 + 2)),  # read ci, xV, u, d_acts; write d_xV, d_ci
    }
    dom = max((n for n in cat_ms if n in work), key=cat_ms.get)
    kind, amount = work[dom]
    launches = cat_n[dom]
    roof = roofline(kind, amount / launches, cat_ms[dom] / launches, dom, launches, pmc_traffic(LLAMA, dom))
    res = {
        "tokens": N, "ms_per_step": ms_per_step,
        "config": {"workload": LLAMA, "batch": B, "seq_len": T, "d_model": d, "heads": H, "kv_heads": KV,
                   "d_mlp": f, "vocab": V, "layers": Ln, "C": dict(C), "imp_min": "p=2",
                   "recon": "kl(clean || masked), streamed over 3 vocab chunks", "mask_draw":
                   "threefry bf16 (partitionable)", "delta_channel": cfg["use_delta"], "attention": "frozen, causal"},
        "step_flops": sum(gf.values()), "phases_ms": cat_ms, "launches_per_step": cat_n, "roofline": roof,
        "reference_rule_flops": gf["gemm_fwd"] + gf["gemm_dx"] + gf["gemm_dw"],
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = lm_cpu_baseline(cfg, args.cpu_tokens)
    return res


def main():
    if "--rocprof-summary" in sys.argv:
        i = sys.argv.index("--rocprof-summary")
        print(rocprof_summary(sys.argv[i + 1], sys.argv[i + 2]))
        return
    if "--rocprof-csv-summary" in sys.argv:
        i = sys.argv.index("--rocprof-csv-summary")
        print(rocprof_csv_summary(sys.argv[i + 1], sys.argv[i + 2]))
        return
    if "--copy-calibration" in sys.argv:
        copy_calibration()
        return
    if "--pmc-traffic-summary" in sys.argv:
        i = sys.argv.index("--pmc-traffic-summary")
        print(pmc_traffic_summary(sys.argv[i + 1], sys.argv[i + 2:]), end="")
        return
    if "--pmc-l2-summary" in sys.argv:
        i = sys.argv.index("--pmc-l2-summary")
        print(pmc_l2_summary(sys.argv[i + 1], sys.argv[i + 2]), end="")
        return
    if "--pmc-mfma-summary" in sys.argv:
        i = sys.argv.index("--pmc-mfma-summary")
        print(pmc_mfma_summary(sys.argv[i + 1], sys.argv[i + 2], sys.argv[i + 3]))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=MOE, choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-tokens", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU (one MI355X); --gpus {args.gpus} is not run. "
              "How the path would shard is a design note, not a measurement.", file=sys.stderr)
        sys.exit(2)
    if args.cpu_tokens is None:
        args.cpu_tokens = {MOE: 1024, DENSE: 2048, CI_MLP: 512, CI_READOUT: 256, PPGD_DENSE: 256,
                           KL_STREAM: 64, LLAMA: 128}.get(args.workload, 0)
    if args.workload == MOE:
        res = run_moe(args)
    elif args.workload == LLAMA:
        res = run_llama(args)
    elif args.workload in (TMS, RESID):
        res = run_toy(args)
    elif args.workload == DENSE:
        res = run_dense(args)
    elif args.workload in (FAITH_DENSE, FAITH_MOE):
        res = run_faith(args)
    elif args.workload == PPGD_DENSE:
        res = run_ppgd(args)
    elif args.workload == PPGD_LLAMA:
        res = run_ppgd_llama(args)
    elif args.workload == PPGD_MOE:
        res = run_ppgd_moe(args)
    elif args.workload == KL_STREAM:
        res = run_kl(args)
    elif args.workload == GEMM_MOE:
        res = run_gemm_moe(args)
    elif args.workload == GEMM_LM:
        res = run_gemm_lm(args)
    else:
        res = run_ci(args)
    ms = res["ms_per_step"]
    faith = args.workload in (FAITH_DENSE, FAITH_MOE)
    fp32_work = faith or args.workload in (TMS, RESID)
    out = {
        "metric": METRIC,
        "value": res["tokens"] / (ms * 1e-3),
        "unit": "matrices/s" if faith else "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if fp32_work else "bf16",
        "data": "synthetic (seeded torch.randn / torch.rand of the named shapes; random-init target and components)",
        "config": res["config"],
        "step_tflops": res["step_flops"] / (ms * 1e-3) / 1e12,
        "step_mfma_frac": res["step_flops"] / (ms * 1e-3) / (PEAK_FP32_MFMA if fp32_work else PEAK_BF16_FLOPS),
        "phases_ms": res["phases_ms"],
        "roofline": res["roofline"],
    }
    if "launches_per_step" in res:
        out["launches_per_step"] = res["launches_per_step"]
    if "tflops" in res:
        out["tflops_per_product"] = res["tflops"]
    for key in ("hipblaslt_tflops", "max_rel_diff_vs_hipblaslt", "dense_equivalents"):
        if key in res:
            out[key] = res[key]
    if "reference_rule_flops" in res:
        out["reference_rule_tflops"] = res["reference_rule_flops"] / (ms * 1e-3) / 1e12
    if "cpu_baseline" in res:
        out["cpu_baseline"] = res["cpu_baseline"]
    print(json.dumps(out))


if __name__ == "__main__":
    main()
