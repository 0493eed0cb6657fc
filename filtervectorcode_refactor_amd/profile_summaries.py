"""Writes the committed profile summaries under profiles/ from a rocprofv3 run's output.

  python -m filtervectorcode_refactor_amd.profile_summaries trace <config> <dir>
      <dir>/trace/t_kernel_stats.csv, t_kernel_trace.csv and <dir>/trace.log (the bench
      line) of `rocprofv3 --kernel-trace --stats ... -- python3 bench.py --config <config>
      --steps S --warmup 1 --no-cpu-baseline`  ->  profiles/select_<config>_kernel_trace.md
  python -m filtervectorcode_refactor_amd.profile_summaries counters <dir>
      <dir>/pmc_{A,B,C}/p_counter_collection.csv of three `rocprofv3 --pmc` passes over
      `bench.py --config cfg2 --steps 1 --warmup 0 --no-cpu-baseline`
      ->  profiles/select_cfg2_counters.md
  python -m filtervectorcode_refactor_amd.profile_summaries traffic <config> <dir>
      <dir>/{FETCH_SIZE,WRITE_SIZE}/p_counter_collection.csv of two `rocprofv3 --pmc`
      passes over `bench.py --config <config> --steps 1 --warmup 0 --no-cpu-baseline
      --calib-copy`  ->  profiles/traffic_select_cross_<config>.txt

Every summary records the digest of the device and launch sources it was measured on
(bench.kernel_source_digest), so a stale one can be told apart.
"""
from __future__ import annotations

import collections
import csv
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

PASSES = {
    "A": "GRBM_GUI_ACTIVE SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS "
         "SQ_INSTS_SALU SQ_VALU_MFMA_BUSY_CYCLES",
    "B": "GRBM_GUI_ACTIVE SQ_VALU_MFMA_COEXEC_CYCLES SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT SQ_WAIT_INST_LDS "
         "SQ_WAIT_INST_ANY SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_ANY",
    "C": "GRBM_GUI_ACTIVE SQ_INSTS_VMEM_RD SQ_INST_CYCLES_VMEM_RD SQ_ACTIVE_INST_VMEM SQ_INSTS_BRANCH SQ_WAIT_ANY "
         "SQ_INSTS_SMEM SQ_ACTIVE_INST_MISC TCC_HIT TCC_MISS",
}
N_XCD = 8            # GRBM_GUI_ACTIVE adds the busy cycles of the eight XCDs
N_SIMD = 256 * 4     # SIMDs of the MI355X
BF16_PEAK = 2.5e15


def _short(name: str) -> str:
    n = name.replace("void ", "").replace("(anonymous namespace)::", "")
    if ">(" in n:
        n = n[: n.index(">(") + 1]
    elif "(" in n:
        n = n[: n.index("(")]
    if "rocprim" in n:
        n = "rocprim " + ("init_lookback_scan_state_kernel" if "init_lookback" in n else "scan kernel (hipCUB ExclusiveSum)")
    return n


def _bench_line(path):
    return json.loads([l for l in open(path) if l.startswith("{")][-1])


def trace(cfg: str, d: str):
    import bench
    from filtervectorcode_refactor_amd import datasets as D
    C = D.CONFIGS[cfg]
    stats = list(csv.DictReader(open(os.path.join(d, "trace", "t_kernel_stats.csv"))))
    tr = list(csv.DictReader(open(os.path.join(d, "trace", "t_kernel_trace.csv"))))
    B = _bench_line(os.path.join(d, "trace.log"))
    rl, bd, cf = B["roofline"], B["breakdown"], B["config"]
    steps, warm = B["steps"], B["warmup"]
    sel = sorted((r for r in tr if "ung_select_kernel<8" in r["Kernel_Name"]), key=lambda r: int(r["Start_Timestamp"]))
    timed = sel[warm: warm + steps]
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6 for r in timed]
    tavg = sum(dur) / len(dur)
    f = rl["mfma_bf16_flops_per_launch"]
    out = [f"# Kernel trace — {cfg} ({C.n:,} x {C.dim} fp32, cross k={C.k_cross} + intra K={C.k_intra}), MI355X", "",
           "Command (from the repository root on the MI355X box):", "",
           f"    rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/meas/{cfg}/trace -o t -- \\",
           f"        python3 bench.py --config {cfg} --steps {steps} --warmup {warm} --no-cpu-baseline", "",
           "Summary (`t_kernel_stats.csv`; durations in microseconds; the run also holds the drop-in calls",
           "with host output and the parity check after the timed steps):", "",
           "| kernel | calls | total us | average us | % |", "|---|---:|---:|---:|---:|"]
    for r in stats:
        out.append(f"| `{_short(r['Name'])}` | {int(r['Calls'])} | {float(r['TotalDurationNs']) / 1e3:.1f} | "
                   f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['Percentage']):.2f} |")
    out += ["",
            f"Cross select (`{_short(sel[0]['Kernel_Name'])}`), the {steps} timed steps' dispatches "
            f"(dispatches {warm + 1}-{warm + steps} of the kernel in the per-dispatch trace `t_kernel_trace.csv`): "
            f"{tavg:.3f} ms on average (min {min(dur):.3f}, max {max(dur):.3f}); the bench's HIP-event average of the "
            f"same launches (`roofline.avg_launch_ms`) is {rl['avg_launch_ms']:.3f} ms "
            f"({abs(tavg - rl['avg_launch_ms']) / rl['avg_launch_ms'] * 100:.1f} % apart).",
            f"Per launch: 3 bf16 MFMA passes, 2 * 3 * dp * P_cross = {f:.4g} FLOP: {f / tavg / 1e9:.0f} TFLOP/s from the "
            f"trace = {f / tavg / 1e9 / (BF16_PEAK / 1e12) * 100:.1f} % of the 2.5 PFLOP/s dense bf16 peak; the line's "
            f"`roofline` ({rl['bound']}) frac is {rl['frac']}."]
    out += ["", f"Bench line of this run: ms_per_step {B['ms_per_step']}, value {B['value']:.4g} {B['unit']}; "
            f"cross select {bd['cross_select_ms']} ms, merge {bd['cross_merge_ms']} ms, additional edges "
            f"{bd['additional_wall_ms']} ms, intra select {bd['intra_select_ms']} ms (in the step, on the second stream "
            f"beside the cross merge and the additional edges), intra merge {bd['intra_merge_ms']} ms.", "",
            f"kernel_source_sha256: {bench.kernel_source_digest()}"]
    path = os.path.join(ROOT, "profiles", f"select_{cfg}_kernel_trace.md")
    open(path, "w").write("\n".join(out) + "\n")
    print("wrote", path)


def counters(d: str):
    import bench
    data = collections.OrderedDict()
    for p in "ABC":
        rows = list(csv.DictReader(open(os.path.join(d, f"pmc_{p}", "p_counter_collection.csv"))))
        for key, label in (("ung_select_kernel<8", "cross select"), ("ung_knn_select_kernel", "intra select"),
                           ("ung_merge_kernel<false>", "merge")):
            hit = [r for r in rows if key in r["Kernel_Name"]]
            first = min(int(r["Dispatch_Id"]) for r in hit)
            e = data.setdefault(label, {"name": _short(hit[0]["Kernel_Name"]), "dur": {}, "disp": {}})
            for r in hit:
                if int(r["Dispatch_Id"]) == first:
                    e[r["Counter_Name"]] = float(r["Counter_Value"])
                    e["dur"][p] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6
                    e["disp"][p] = first
    cols = list(data)
    out = ["# Counters — cfg2 (1,000,000 x 128): cross select, intra (mid-group) select, merge; MI355X", "",
           "Commands (repository root, MI355X box; one counter block per run; the first dispatch of each",
           "kernel in the run; counter collection serializes the dispatches, so each kernel ran alone):", ""]
    for p, cs in PASSES.items():
        out.append(f"    rocprofv3 --pmc {cs} --output-format csv -d gpurun_out/meas/cfg2/pmc_{p} -o p -- \\")
        out.append("        python3 bench.py --config cfg2 --steps 1 --warmup 0 --no-cpu-baseline")
    out += ["", "| counter | " + " | ".join(f"{c} `{data[c]['name']}`" for c in cols) + " |",
            "|---|" + "---:|" * len(cols)]
    names = sorted({k for c in cols for k in data[c] if k.isupper() or k.startswith("SQ_") or k.startswith("TCC") or
                    k.startswith("GRBM")})
    out.append("| duration (ms), passes A/B/C | " + " | ".join(
        "/".join(f"{data[c]['dur'][p]:.3f}" for p in "ABC") for c in cols) + " |")
    for n in names:
        out.append(f"| {n} | " + " | ".join(f"{data[c].get(n, float('nan')):,.0f}" for c in cols) + " |")
    out += ["", "Derived (pass A's duration and GRBM_GUI_ACTIVE; the eight XCDs' busy cycles are summed, so the",
            "clock is GRBM_GUI_ACTIVE / 8 / duration; MFMA cycles per instruction = SQ_VALU_MFMA_BUSY_CYCLES /",
            "SQ_INSTS_MFMA; SQ_INSTS_VALU counts the MFMAs too; a VALU instruction of a wave64 takes four",
            "cycles of its SIMD):", "",
            "| quantity | " + " | ".join(cols) + " |", "|---|" + "---:|" * len(cols)]

    def row(label, fn):
        vals = []
        for c in cols:
            try:
                vals.append(fn(data[c]))
            except (KeyError, ZeroDivisionError):
                vals.append("-")
        out.append(f"| {label} | " + " | ".join(vals) + " |")

    clock = lambda e: e["GRBM_GUI_ACTIVE"] / N_XCD / (e["dur"]["A"] * 1e-3)
    avail = lambda e: N_SIMD * clock(e) * e["dur"]["A"] * 1e-3
    row("clock (GHz)", lambda e: f"{clock(e) / 1e9:.3f}")
    row("MFMA busy / SIMD cycles", lambda e: f"{e['SQ_VALU_MFMA_BUSY_CYCLES'] / avail(e) * 100:.1f} %")
    row("cycles per MFMA", lambda e: f"{e['SQ_VALU_MFMA_BUSY_CYCLES'] / e['SQ_INSTS_MFMA']:.1f}")
    row("VALU (non-MFMA) per MFMA", lambda e: f"{(e['SQ_INSTS_VALU'] - e['SQ_INSTS_MFMA']) / e['SQ_INSTS_MFMA']:.2f}")
    row("VALU (non-MFMA) cycles / SIMD cycles", lambda e: f"{4 * (e['SQ_INSTS_VALU'] - e['SQ_INSTS_MFMA']) / avail(e) * 100:.1f} %")
    row("MFMA-VALU co-execution / MFMA busy", lambda e: f"{e['SQ_VALU_MFMA_COEXEC_CYCLES'] / e['SQ_VALU_MFMA_BUSY_CYCLES'] * 100:.1f} %")
    row("LDS bank-conflict cycles / LDS active", lambda e: f"{e['SQ_LDS_BANK_CONFLICT'] / e['SQ_LDS_IDX_ACTIVE'] * 100:.1f} %")
    row("wave cycles waiting on LDS", lambda e: f"{e['SQ_WAIT_INST_LDS'] / e['SQ_WAVE_CYCLES'] * 100:.1f} %")
    row("wave cycles waiting (any instruction)", lambda e: f"{e['SQ_WAIT_INST_ANY'] / e['SQ_WAVE_CYCLES'] * 100:.1f} %")
    row("L2 hit rate (TCC)", lambda e: f"{e['TCC_HIT'] / (e['TCC_HIT'] + e['TCC_MISS']) * 100:.1f} %")
    out += ["", f"kernel_source_sha256: {bench.kernel_source_digest()}"]
    path = os.path.join(ROOT, "profiles", "select_cfg2_counters.md")
    open(path, "w").write("\n".join(out) + "\n")
    print("wrote", path)


def traffic(cfg: str, d: str):
    import bench
    from filtervectorcode_refactor_amd import datasets as D
    C = D.CONFIGS[cfg]

    def read(counter):
        rows = list(csv.DictReader(open(os.path.join(d, counter, "p_counter_collection.csv"))))
        calib = [r for r in rows if "copyBuffer" in r["Kernel_Name"] and int(r["Grid_Size"]) >= 131072]
        sel = sorted((r for r in rows if "ung_select_kernel<8" in r["Kernel_Name"]), key=lambda r: int(r["Dispatch_Id"]))
        assert len(calib) == 1, [r["Grid_Size"] for r in rows if "copyBuffer" in r["Kernel_Name"]]
        s = sel[0]
        dur = (int(s["End_Timestamp"]) - int(s["Start_Timestamp"])) / 1e6
        return float(calib[0]["Counter_Value"]), float(s["Counter_Value"]), dur, s["Kernel_Name"], s["Dispatch_Id"], len(sel)

    fc, fk, fd, name, fdisp, nsel = read("FETCH_SIZE")
    wc, wk, wd, _, wdisp, _ = read("WRITE_SIZE")
    fs, ws = 1048576.0 / fc, 1048576.0 / wc
    fb, wb = fk * 1024.0 * fs, wk * 1024.0 * ws
    cmd = ("rocprofv3 --pmc {c} --output-format csv -d gpurun_out/meas/" + cfg + "/{c} -o p -- python3 bench.py "
           "--config " + cfg + " --steps 1 --warmup 0 --no-cpu-baseline --calib-copy")
    out = f"""HBM traffic of one cross select launch ({_short(name)}), {cfg} {C.n:,} x {C.dim}

Commands (repository root, MI355X box; one counter block per pass):
  {cmd.format(c='FETCH_SIZE')}
  {cmd.format(c='WRITE_SIZE')}

Calibration (--calib-copy: one 1 GiB device-to-device hipMemcpy, runtime blit kernel
__amd_rocclr_copyBuffer, 1,048,576 KiB read and 1,048,576 KiB written):
  FETCH_SIZE reads {fc:,.1f} KiB -> scale {fs:.4f} (1,048,576 / {fc:,.1f})
  WRITE_SIZE reads {wc:,.1f} KiB -> scale {ws:.4f}

Select kernel (the first of each pass's {nsel} cross select dispatches: Dispatch_Id {fdisp} in the
FETCH_SIZE pass, {wdisp} in the WRITE_SIZE pass):
  FETCH_SIZE {fk:,.1f} KiB x {fs:.4f} = {int(fb):,} B
  WRITE_SIZE {wk:,.1f} KiB x {ws:.4f} = {int(wb):,} B
  duration {fd:.2f} ms (FETCH pass) / {wd:.2f} ms (WRITE pass), counters serialize the dispatches

traffic_bytes_per_launch: {int(round(fb + wb))}
kernel_source_sha256: {bench.kernel_source_digest()}
"""
    path = os.path.join(ROOT, "profiles", f"traffic_select_cross_{cfg}.txt")
    open(path, "w").write(out)
    print("wrote", path)


if __name__ == "__main__":
    what = sys.argv[1]
    if what == "trace":
        trace(sys.argv[2], sys.argv[3])
    elif what == "counters":
        counters(sys.argv[2])
    elif what == "traffic":
        traffic(sys.argv[2], sys.argv[3])
    else:
        raise SystemExit(__doc__)
