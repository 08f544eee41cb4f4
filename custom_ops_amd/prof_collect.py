"""Collect the rocprofv3 evidence for one configuration and write text summaries.

    python -m custom_ops_amd.prof_collect --config cfg2 --out prof_out
    python -m custom_ops_amd.prof_collect --config cfg2 --stall --out prof_out
    python -m custom_ops_amd.prof_collect --bench --out prof_out

Runs, each as its own rocprofv3 process under a hard time limit (this process
never touches the GPU itself):
  1. --kernel-trace --stats          per-kernel average duration
  2. --pmc FETCH_SIZE                HBM read KiB per dispatch
  3. --pmc WRITE_SIZE                HBM write KiB per dispatch
  4. --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_MFMA GRBM_GUI_ACTIVE
  5. --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS GRBM_GUI_ACTIVE
  6. --pmc FETCH_SIZE with the mask's strides set to 0 (prof_workload
     --mask-bcast): the FETCH_SIZE difference against pass 2 is the HBM
     traffic of the mask stream, which gives its counted GB/s
The workload (custom_ops_amd.prof_workload) first runs y = 2·x over a 512 MiB
fp32 buffer (5 dispatches of one elementwise kernel that reads and writes
512 MiB each); its FETCH_SIZE / WRITE_SIZE against the known 512 MiB give the
calibration factor applied to the attention kernel's counters.
rocprofv3 reports GRBM_GUI_ACTIVE summed over the 8 XCDs; the per-XCD active
cycles (GUI / 8) are the kernel's cycle count at the clock it ran at.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import shutil
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
COPY_MIB = 512

PASSES = {
    "trace": ["--kernel-trace", "--stats"],
    "fetch": ["--pmc", "FETCH_SIZE"],
    "write": ["--pmc", "WRITE_SIZE"],
    "mfma": ["--pmc", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_MFMA",
             "GRBM_GUI_ACTIVE"],
    "lds": ["--pmc", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS",
            "GRBM_GUI_ACTIVE"],
    "fetch_bcast": ["--pmc", "FETCH_SIZE"],
}


# --stall: wave-state counters of the attention kernel (three passes, each
# within the per-block limits of one rocprofv3 --pmc run)
STALL_PASSES = {
    "stall1": ["--pmc", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
               "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_MISC"],
    "stall2": ["--pmc", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_SCA",
               "SQ_INST_CYCLES_SALU", "SQ_LDS_IDX_ACTIVE", "SQ_LDS_ADDR_CONFLICT",
               "SQ_LDS_DATA_FIFO_FULL", "SQ_LDS_CMD_FIFO_FULL"],
    "stall3": ["--pmc", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_ACTIVE_INST_VALU2",
               "SQ_LDS_UNALIGNED_STALL", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES",
               "GRBM_GUI_ACTIVE"],
}


COLD = False   # --cold: every counted launch after a cache flush
VARIANT = ""   # --variant: kernel-variant fields passed to every call


def workload_cmd(cfg: str, iters: int, bcast: bool = False) -> list[str]:
    return [sys.executable, "-m", "custom_ops_amd.prof_workload", "--config", cfg, "--iters",
            str(iters), "--copy-mib", str(COPY_MIB), *(["--mask-bcast"] if bcast else []),
            *(["--cold"] if COLD else []), *(["--variant", VARIANT] if VARIANT else [])]


def rocprof_cmd(name: str, outdir: str, cfg: str, iters: int) -> list[str]:
    if name == "bench":
        return ["rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv", "-d", outdir, "--",
                sys.executable, os.path.join(ROOT, "bench.py"), "--no-cpu", "--no-configs"]
    args = PASSES.get(name) or STALL_PASSES[name]
    return ["rocprofv3", *args, "--output-format", "csv", "-d", outdir, "--",
            *workload_cmd(cfg, iters, bcast=name.endswith("_bcast"))]


def run_pass(name: str, outdir: str, cfg: str, iters: int) -> str:
    d = os.path.join(outdir, "raw", name)
    shutil.rmtree(d, ignore_errors=True)
    os.makedirs(d, exist_ok=True)
    cmd = rocprof_cmd(name, d, cfg, iters)
    env = dict(os.environ, TMPDIR="/tmp", PYTHONPATH=ROOT)
    print("[prof]", " ".join(cmd), flush=True)
    res = subprocess.run(["timeout", "-s", "KILL", "90", *cmd], cwd="/tmp", env=env,
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"pass {name} failed ({res.returncode}):\n{res.stdout[-2000:]}\n"
                           f"{res.stderr[-2000:]}")
    return d


def rows(d: str, suffix: str) -> list[dict]:
    out = []
    for f in glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True):
        with open(f, newline="") as fh:
            out.extend(csv.DictReader(fh))
    return out


def is_attn(name: str) -> bool:
    return "fa_fwd_kernel" in name


def is_combine(name: str) -> bool:
    return "fa_combine_kernel" in name


def is_map(name: str) -> bool:
    return "mask_stage_kernel" in name   # the mask pre-pass (staged copy and/or live-tile map)


def is_copy(name: str) -> bool:
    return "MulFunctor" in name


def counter_means(d: str, pred) -> dict[str, float]:
    """Mean over matching dispatches of each counter (summed over its instances)."""
    per = {}
    for r in rows(d, "counter_collection.csv"):
        if not pred(r["Kernel_Name"]):
            continue
        key = (r.get("Dispatch_Id") or r.get("Correlation_Id"), r["Counter_Name"])
        per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    acc = {}
    for (_, cname), v in per.items():
        acc.setdefault(cname, []).append(v)
    return {k: sum(v) / len(v) for k, v in acc.items()}


def write_summary(path: str, title: str, cmds: list[str], body: list[str]) -> None:
    lines = [title, "", "commands (run from the repository root; each pass is its own process):"]
    lines += ["  " + c for c in cmds] + [""] + body
    txt = "\n".join(lines) + "\n"
    with open(path, "w") as f:
        f.write(txt)
    print(txt, flush=True)


def bench_main(args) -> None:
    """Kernel trace of bench.py's own timed run (cfg2): the attention kernel's
    average over every launch, and over the cold steps alone (the launches
    that directly follow the bench's flush read-back), for comparison with the
    bench line's event-timed roofline figure."""
    d = run_pass("bench", args.out, "", 0)
    stats = rows(d, "kernel_stats.csv")
    trace = sorted(rows(d, "kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    cold = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            for i, r in enumerate(trace)
            if is_attn(r["Kernel_Name"]) and i and "reduce_kernel" in trace[i - 1]["Kernel_Name"]]
    body = ["kernel trace (--stats):",
            f"  {'name':<70} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9}"]
    for r in stats:
        body.append(f"  {r['Name'][:70]:<70} {int(r['Calls']):>6} {float(r['AverageNs'])/1e3:>9.2f} "
                    f"{float(r['MinNs'])/1e3:>9.2f} {float(r['MaxNs'])/1e3:>9.2f}")
    cs = sorted(cold)
    body += ["", "cold steps (attention launches right after the flush read-back):",
             f"  count                              {len(cold)}",
             f"  mean_us                            {sum(cold) / max(1, len(cold)):.6g}",
             f"  median_us                          {cs[len(cs) // 2] if cs else float('nan'):.6g}",
             f"  min_us                             {cs[0] if cs else float('nan'):.6g}",
             f"  max_us                             {cs[-1] if cs else float('nan'):.6g}"]
    write_summary(os.path.join(args.out, "bench_fa_fwd_kernel_cfg2_trace.txt"),
                  "# rocprofv3 summary: bench.py --no-cpu --no-configs (cfg2), kernel trace",
                  ["python -m custom_ops_amd.prof_collect --bench",
                   "cd /tmp && TMPDIR=/tmp PYTHONPATH=<repo> " + " ".join(rocprof_cmd("bench", "<out>/raw/bench", "", 0))],
                  body)


def stall_main(args, cfg) -> None:
    """Wave-state counters: where the attention kernel's waves spend their time."""
    dirs = {p: run_pass(p, args.out, cfg.name, args.iters) for p in STALL_PASSES}
    m = {}
    for d in dirs.values():
        m.update(counter_means(d, is_attn))
    wc = m["SQ_WAVE_CYCLES"]
    body = ["counters (mean per dispatch, summed over the device):"]
    body += [f"  {k:<28} {m[k]:.4g}" for k in sorted(m)]
    body += ["", "as a share of SQ_WAVE_CYCLES (wave-resident time):"]
    for k in ("SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_SCA",
              "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_MISC", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
              "SQ_WAIT_INST_LDS", "SQ_LDS_IDX_ACTIVE"):
        body.append(f"  {k:<28} {m[k] / wc:.3f}")
    gui = m["GRBM_GUI_ACTIVE"] / 8
    body += ["", f"  MFMA busy per SIMD / kernel cycles   {m['SQ_VALU_MFMA_BUSY_CYCLES'] / 1024 / gui:.3f}"]
    write_summary(os.path.join(args.out, f"stall_fa_fwd_kernel_{cfg.name}.txt"),
                  f"# rocprofv3 wave-state counters: fa_fwd_kernel on {cfg.name} "
                  f"(B={cfg.B} H={cfg.H} Hk={cfg.Hk} Sq={cfg.Sq} Sk={cfg.Sk} d={cfg.d})",
                  [f"python -m custom_ops_amd.prof_collect --config {cfg.name} --stall --iters {args.iters}"]
                  + ["cd /tmp && TMPDIR=/tmp PYTHONPATH=<repo> timeout -s KILL 90 " +
                     " ".join(rocprof_cmd(p, f"<out>/raw/{p}", cfg.name, args.iters)) for p in STALL_PASSES],
                  body)


POWER_LOADS = [("cfg2", ["--config", "cfg2"]), ("cfg3", ["--config", "cfg3"]), ("cfg4", ["--config", "cfg4"]),
               ("cfg5", ["--config", "cfg5"])]


def smi_sample() -> tuple[float | None, list[float]]:
    """Socket power (W) and the XCD graphics clocks (MHz) from amd-smi."""
    res = subprocess.run(["timeout", "20", "amd-smi", "metric", "-p", "-c"], capture_output=True, text=True)
    watts, clocks, in_gfx = None, [], False
    for line in res.stdout.splitlines():
        t = line.strip()
        if t.startswith("SOCKET_POWER:"):
            try:
                watts = float(t.split()[1])
            except (IndexError, ValueError):
                pass
        elif t.startswith("GFX_"):
            in_gfx = True
        elif t.endswith(":") and not t.startswith("GFX_"):
            in_gfx = t.startswith("GFX")
        elif in_gfx and t.startswith("CLK:"):
            try:
                clocks.append(float(t.split()[1]))
            except (IndexError, ValueError):
                pass
            in_gfx = False
    return watts, clocks


def power_main(args) -> None:
    """Steady-state socket power and XCD clocks: each workload runs back to
    back for --loop-s seconds in its own process; amd-smi is sampled twice in
    the second half."""
    from custom_ops_amd.workloads import CONFIGS
    env = dict(os.environ, PYTHONPATH=ROOT)
    idle_w, idle_c = smi_sample()
    body = [f"idle: socket {idle_w} W", "",
            f"  {'workload':<12} {'rate':>22} {'socket_W':>9} {'xcd_clock_MHz(min/mean/max)':>30}"]
    rates = {}
    for name, extra in POWER_LOADS:
        cmd = [sys.executable, "-m", "custom_ops_amd.prof_workload", *extra, "--loop-s", str(args.loop_s)]
        print("[power]", " ".join(cmd), flush=True)
        proc = subprocess.Popen(["timeout", "-s", "KILL", str(int(args.loop_s) + 90), *cmd], env=env,
                                stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        time.sleep(args.loop_s * 0.55 + 3)
        samples = [smi_sample()]
        time.sleep(1.0)
        samples.append(smi_sample())
        out, _ = proc.communicate()
        if proc.returncode != 0:
            raise RuntimeError(f"{name} failed ({proc.returncode}):\n{out[-2000:]}")
        last = [l for l in out.splitlines() if l.startswith("prof_workload")][-1]
        watts = [w for w, _ in samples if w is not None]
        clocks = [c for _, cs in samples for c in cs[:8]]
        us = float(last.split(",")[-1].split()[0])
        tflops = CONFIGS[name].flops / (us * 1e-6) / 1e12
        rate = f"{us:.1f} us = {tflops:.0f} TFLOP/s"
        rates[name] = tflops
        w = max(watts) if watts else float("nan")
        cl = (f"{min(clocks):.0f}/{sum(clocks) / len(clocks):.0f}/{max(clocks):.0f}" if clocks else "n/a")
        body.append(f"  {name:<12} {rate:>22} {w:>9.0f} {cl:>30}")
    body += ["", "derived:"] + [f"  {n} / 2500 TFLOP/s{'':<17} {r / 2500:.3f}" for n, r in rates.items()]
    write_summary(os.path.join(args.out, "power_clocks.txt"),
                  "# socket power and XCD clocks under each workload (amd-smi, steady state)",
                  [f"python -m custom_ops_amd.prof_collect --power --loop-s {args.loop_s}"]
                  + ["python -m custom_ops_amd.prof_workload " + " ".join(e) + f" --loop-s {args.loop_s}"
                     for _, e in POWER_LOADS]
                  + ["amd-smi metric -p -c   (sampled twice in the second half of each run)"],
                  body)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--out", default=os.path.join(ROOT, "prof_out"))
    ap.add_argument("--stall", action="store_true", help="wave-state counters instead")
    ap.add_argument("--cold", action="store_true",
                    help="flush the caches before every counted launch (the bench's cold launches)")
    ap.add_argument("--variant", default="",
                    help="kernel-variant fields for every call, e.g. order=1 (summaries get a suffix)")
    ap.add_argument("--bench", action="store_true", help="kernel trace of bench.py's timed run instead")
    ap.add_argument("--power", action="store_true", help="socket power and clocks per workload instead")
    ap.add_argument("--loop-s", type=float, default=10.0, help="--power: seconds per workload")
    args = ap.parse_args()
    args.out = os.path.abspath(args.out)      # the passes run with cwd=/tmp
    global COLD, VARIANT
    COLD = args.cold
    VARIANT = args.variant
    os.makedirs(args.out, exist_ok=True)
    sys.path.insert(0, ROOT)
    from custom_ops_amd.workloads import CONFIGS
    if args.bench:
        bench_main(args)
        return
    if args.power:
        power_main(args)
        return
    cfg = CONFIGS[args.config]
    if args.stall:
        stall_main(args, cfg)
        return

    dirs = {p: run_pass(p, args.out, cfg.name, args.iters) for p in PASSES}

    stats = rows(dirs["trace"], "kernel_stats.csv")
    attn = [r for r in stats if is_attn(r["Name"])]
    if not attn:
        raise RuntimeError("no fa_fwd_kernel dispatch in the kernel trace")
    avg_ns = float(attn[0]["AverageNs"])
    comb = [r for r in stats if is_combine(r["Name"])]
    lmap = [r for r in stats if is_map(r["Name"])]

    fetch_copy = counter_means(dirs["fetch"], is_copy).get("FETCH_SIZE")
    write_copy = counter_means(dirs["write"], is_copy).get("WRITE_SIZE")
    fetch = counter_means(dirs["fetch"], is_attn)["FETCH_SIZE"]
    write = counter_means(dirs["write"], is_attn)["WRITE_SIZE"]
    kib = COPY_MIB * 1024
    f_fac = kib / fetch_copy if fetch_copy else None
    w_fac = kib / write_copy if write_copy else None
    traffic = None
    if f_fac and w_fac:
        traffic = (fetch * f_fac + write * w_fac) * 1024
    fetch_map = counter_means(dirs["fetch"], is_map).get("FETCH_SIZE")
    fetch_comb = counter_means(dirs["fetch"], is_combine).get("FETCH_SIZE")
    write_comb = counter_means(dirs["write"], is_combine).get("WRITE_SIZE")
    fetch_b = counter_means(dirs["fetch_bcast"], is_attn)["FETCH_SIZE"]
    mask_alg = cfg.B * cfg.Sq * cfg.Sk * 2
    # The broadcast call (mask strides 0) is a like-for-like comparison only
    # when the mask's rows are 16-byte aligned already: with unaligned rows
    # (Sk % 8 != 0) the strides-0 call takes the aligned mask path and skips
    # the live-tile map, so the difference would not be the mask stream.
    aligned = cfg.Sk % 8 == 0
    mask_counted = (fetch - fetch_b) * f_fac * 1024 if (f_fac and aligned) else None
    mf = counter_means(dirs["mfma"], is_attn)
    ld = counter_means(dirs["lds"], is_attn)
    simds, xcds = 256 * 4, 8
    gui = mf["GRBM_GUI_ACTIVE"] / xcds
    mfma_util = 100 * mf["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * simds)
    mfma_flops = mf.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0) * 512
    bank_conf = ld["SQ_LDS_BANK_CONFLICT"] / max(1.0, ld["SQ_LDS_IDX_ACTIVE"])

    kname = attn[0]["Name"]
    stem = (f"fa_fwd_kernel_{cfg.name}" + ("_cold" if COLD else "")
            + ("_" + VARIANT.replace("=", "").replace(",", "_") if VARIANT else ""))
    # The counted launches are the last --iters of each kernel in the trace
    # (the clock-settle launches come first): their mean duration, and for
    # a launch sequence the mean of (end of its last kernel - start of the
    # attention kernel), i.e. including the gap to a map / combine kernel.
    trace = sorted(rows(dirs["trace"], "kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))

    def counted(pred):
        ds = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in trace if pred(r["Kernel_Name"])]
        ds = ds[-args.iters:]
        return sum(ds) / len(ds) if ds else None

    ours = [r for r in trace if "mi355fa::" in r["Kernel_Name"]]
    spans, i = [], 0
    while i < len(ours):            # a call: [mask pre-pass] attention [combine]
        j = i
        while j < len(ours) and not is_attn(ours[j]["Kernel_Name"]):
            j += 1
        if j == len(ours):
            break
        start = int(ours[i]["Start_Timestamp"])
        end = int(ours[j]["End_Timestamp"])
        if j + 1 < len(ours) and is_combine(ours[j + 1]["Kernel_Name"]):
            j += 1
            end = int(ours[j]["End_Timestamp"])
        spans.append((end - start) / 1e3)
        i = j + 1
    spans = spans[-args.iters:]
    mask_bytes = cfg.B * cfg.Sq * cfg.Sk * 2
    summary = {
        "config": cfg.name,
        "kernel": kname,
        "calls": int(attn[0]["Calls"]),
        "avg_duration_us": avg_ns / 1e3,
        "min_duration_us": float(attn[0]["MinNs"]) / 1e3,
        "max_duration_us": float(attn[0]["MaxNs"]) / 1e3,
        "counted_launches": args.iters,
        "counted_avg_us": counted(is_attn),
        "counted_combine_avg_us": counted(is_combine) if comb else None,
        "counted_mask_prepass_avg_us": counted(is_map) if lmap else None,
        "counted_call_span_us": sum(spans) / len(spans) if spans else None,
        "combine_avg_us": float(comb[0]["AverageNs"]) / 1e3 if comb else None,
        "mask_prepass_avg_us": float(lmap[0]["AverageNs"]) / 1e3 if lmap else None,
        "mask_prepass_fetch_bytes": fetch_map * f_fac * 1024 if (fetch_map and f_fac) else None,
        "combine_bytes": ((fetch_comb or 0) * f_fac + (write_comb or 0) * w_fac) * 1024
                         if (comb and f_fac and w_fac) else None,
        "achieved_tflops": cfg.flops / (avg_ns * 1e-9) / 1e12,
        "pct_bf16_peak": 100 * cfg.flops / (avg_ns * 1e-9) / 1e12 / 2500.0,
        "fetch_kib_raw": fetch, "write_kib_raw": write,
        "copy_fetch_kib_raw": fetch_copy, "copy_write_kib_raw": write_copy,
        "fetch_factor": f_fac, "write_factor": w_fac,
        "hbm_bytes_per_launch": traffic,
        "algorithmic_bytes_per_launch": cfg.algorithmic_bytes,
        "hbm_gbps": traffic / (avg_ns * 1e-9) / 1e9 if traffic else None,
        "mask_stream_gbps_algorithmic": mask_bytes / (avg_ns * 1e-9) / 1e9,
        "fetch_kib_raw_mask_bcast": fetch_b,
        "mask_hbm_bytes_counted": mask_counted,
        "mask_hbm_gbps_counted": mask_counted / (avg_ns * 1e-9) / 1e9 if mask_counted else None,
        "mfma_busy_pct": mfma_util,
        "active_cycles_per_xcd": gui,
        "clock_ghz_under_counters": gui / (avg_ns * 1e-9) / 1e9,
        "mfma_bf16_flops_counted": mfma_flops,
        "mfma_insts": mf.get("SQ_INSTS_MFMA"),
        "lds_bank_conflict_cycles": ld["SQ_LDS_BANK_CONFLICT"],
        "lds_active_cycles": ld["SQ_LDS_IDX_ACTIVE"],
        "lds_insts": ld["SQ_INSTS_LDS"],
        "lds_bank_conflict_ratio": bank_conf,
    }
    with open(os.path.join(args.out, f"traffic_{stem}.json"), "w") as f:
        json.dump({"config": cfg.name, "kernel": kname,
                   "hbm_bytes_per_launch": traffic,
                   "fetch_factor": f_fac, "write_factor": w_fac,
                   "avg_duration_us": avg_ns / 1e3}, f, indent=1)
    with open(os.path.join(args.out, f"mask_stream_{stem}.json"), "w") as f:
        json.dump({"config": cfg.name, "kernel": kname,
                   "mask_bytes_algorithmic": mask_alg,
                   "mask_hbm_bytes_counted": mask_counted,
                   "mask_hbm_gbps_counted": (mask_counted / (avg_ns * 1e-9) / 1e9
                                             if mask_counted else None),
                   "fetch_kib_raw": fetch, "fetch_kib_raw_mask_bcast": fetch_b,
                   "fetch_factor": f_fac, "avg_duration_us": avg_ns / 1e3,
                   "source": "rocprofv3 FETCH_SIZE, normal call minus the same call with mask "
                             "strides 0 (custom_ops_amd.prof_collect)"}, f, indent=1)
    lines = [f"# rocprofv3 summary: fa_fwd_kernel on {cfg.name}", ""]
    lines.append(f"workload: {cfg.name} B={cfg.B} H={cfg.H} Hk={cfg.Hk} Sq={cfg.Sq} Sk={cfg.Sk} "
                 f"d={cfg.d} bf16 ({cfg.description}); {args.iters} launches after clock settle"
                 + (", each after a 512 MiB zero + read-back (cold caches)" if COLD else ", back to back"))
    lines.append("")
    lines.append("commands (run from the repository root; each pass is its own process):")
    lines.append(f"  python -m custom_ops_amd.prof_collect --config {cfg.name} --iters {args.iters}"
                 + (" --cold" if COLD else "") + (f" --variant {VARIANT}" if VARIANT else ""))
    for p in PASSES:
        lines.append("  cd /tmp && TMPDIR=/tmp PYTHONPATH=<repo> " +
                     " ".join(rocprof_cmd(p, f"<out>/raw/{p}", cfg.name, args.iters)))
    lines.append("")
    lines.append("kernel trace (--stats), all kernels:")
    lines.append(f"  {'name':<70} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9}")
    for r in stats:
        lines.append(f"  {r['Name'][:70]:<70} {int(r['Calls']):>6} {float(r['AverageNs'])/1e3:>9.2f} "
                     f"{float(r['MinNs'])/1e3:>9.2f} {float(r['MaxNs'])/1e3:>9.2f}")
    lines.append("")
    lines.append("derived:")
    for k, v in summary.items():
        if isinstance(v, float):
            v = f"{v:.6g}"
        lines.append(f"  {k:<34} {v}")
    txt = "\n".join(lines) + "\n"
    with open(os.path.join(args.out, f"{stem}.txt"), "w") as f:
        f.write(txt)
    print(txt, flush=True)


if __name__ == "__main__":
    main()
