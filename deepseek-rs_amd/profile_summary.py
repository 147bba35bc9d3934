"""Summaries of rocprofv3 output for profiles/ (text the benchmark and the
design notes quote).  Reads only CSV files that rocprofv3 wrote (run it with
--output-format csv); runs no GPU code.

  python deepseek-rs_amd/profile_summary.py kernels  OUT DIR  --title T --cmd C
      kernel-time table from DIR/*_kernel_stats.csv
  python deepseek-rs_amd/profile_summary.py traffic  OUT FETCH_DIR WRITE_DIR --config C --path P --title T --cmd C
      HBM bytes per dispatch from one FETCH_SIZE run and one WRITE_SIZE run,
      scaled by the copy kernel of the benchmark's --copy-calibration (a
      256 MiB device copy: 256 MiB read and 256 MiB written)
  python deepseek-rs_amd/profile_summary.py counters OUT DIR [DIR ...] --title T --cmd C
      medians per kernel and counter over the dispatches in DIR/*_counter_collection.csv;
      plus the busy fractions derived() forms from the counters of one run
      (VALU, LDS, LDS bank conflicts, matrix cores, TA stalled by the L1)

Every table row of a dsmoe kernel carries the hash of the code object it was
measured on (`code_object=`), so a summary of an older build is recognisable
as stale (bench.py uses a traffic line only when the hash matches the
current build)."""
import argparse
import csv
import glob
import hashlib
import os
import statistics

HERE = os.path.dirname(os.path.abspath(__file__))
GEMM_PREFIXES = ("dsmoe_gu_grouped", "dsmoe_dn_grouped", "dsmoe_q80_gemm", "dsmoe_q80_combine", "dsmoe_router_tile",
                 "dsmoe_q80_wide", "dsmoe_q80_unpack",
                 "dsmoe_probe")
COPY_KERNEL = "__amd_rocclr_copyBuffer"
COPY_KIB = 256 * 1024  # the calibration copy: 256 MiB read and 256 MiB written
SIMDS, XCDS, CUS = 1024, 8, 256  # MI355X: 256 compute units x 4 SIMDs; GRBM_GUI_ACTIVE is summed over the 8 XCDs


def code_object_hash(kernel, lib_dir=None):
    """First 16 hex digits of the SHA-256 of the code object that holds
    `kernel` (dsmoe_gemm.hsaco for the grouped GEMMs, the batch router and
    the probes, else dsmoe_kernels.hsaco), or None when it is not built."""
    lib_dir = lib_dir or os.path.join(HERE, "lib")
    name = "dsmoe_gemm.hsaco" if kernel.startswith(GEMM_PREFIXES) else "dsmoe_kernels.hsaco"
    f = os.path.join(lib_dir, name)
    if not os.path.exists(f):
        return None
    with open(f, "rb") as fh:
        return hashlib.sha256(fh.read()).hexdigest()[:16]


def _one(pattern):
    files = sorted(glob.glob(pattern))
    if not files:
        raise SystemExit(f"no file matches {pattern}")
    return files[0]


def _header(title, cmd):
    return [f"# {title}", "#", "# command (GPU box, repository root as the working directory):"] + \
           [f"#   {line}" for line in cmd.split(" && ")] + ["#"]


def kernels(out, d, title, cmd):
    rows = list(csv.DictReader(open(_one(os.path.join(d, "*kernel_stats.csv")))))
    lines = _header(title, cmd)
    lines.append(f"{'kernel':34s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s}  code_object")
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        k = r["Name"]
        h = code_object_hash(k) if k.startswith("dsmoe_") else None
        lines.append(f"{k[:34]:34s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} "
                     f"{float(r['MinNs']) / 1e3:10.2f} {float(r['MaxNs']) / 1e3:10.2f}  {h or '-'}")
    open(out, "w").write("\n".join(lines) + "\n")


def _counters(d):
    """{kernel: {counter: [values per dispatch]}} from one counter run."""
    per = {}
    for r in csv.DictReader(open(_one(os.path.join(d, "*counter_collection.csv")))):
        k, c = r["Kernel_Name"], r["Counter_Name"]
        per.setdefault(k, {}).setdefault(c, {})
        per[k][c][r["Dispatch_Id"]] = per[k][c].get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    return {k: {c: list(v.values()) for c, v in cs.items()} for k, cs in per.items()}


def traffic(out, fetch_dir, write_dir, config, path, title, cmd):
    f, w = _counters(fetch_dir), _counters(write_dir)
    med = lambda xs: statistics.median(xs) if xs else 0.0
    # the calibration copies are the largest copy dispatches (the benchmark's
    # other copies move a few KiB of setup data)
    big = lambda xs: [x for x in xs if x >= 0.5 * max(xs)] if xs else []
    cf = med(big(f.get(COPY_KERNEL, {}).get("FETCH_SIZE", [])))
    cw = med(big(w.get(COPY_KERNEL, {}).get("WRITE_SIZE", [])))
    if not cf or not cw:
        raise SystemExit("no calibration copy in the runs (bench.py --copy-calibration)")
    sf, sw = COPY_KIB / cf, COPY_KIB / cw
    lines = _header(title, cmd)
    lines += [f"# calibration: the {COPY_KIB} KiB device copy reads FETCH_SIZE {cf:.1f} KiB and WRITE_SIZE "
              f"{cw:.1f} KiB -> scale factors fetch x{sf:.3f}, write x{sw:.3f}; medians over dispatches", "#",
              f"{'kernel':30s} {'FETCH_KiB':>12s} {'WRITE_KiB':>12s} {'HBM_read_MB':>12s} {'HBM_write_MB':>12s}"]
    mach = []
    for k in sorted(set(f) | set(w)):
        if not k.startswith("dsmoe_") or k == "dsmoe_synth":
            continue
        fk, wk = med(f.get(k, {}).get("FETCH_SIZE", [])), med(w.get(k, {}).get("WRITE_SIZE", []))
        rb, wb = fk * sf * 1024, wk * sw * 1024
        lines.append(f"{k[:30]:30s} {fk:12.1f} {wk:12.1f} {rb / 1e6:12.3f} {wb / 1e6:12.3f}")
        mach.append(f"traffic kernel={k} config={config} path={path} bytes={int(rb + wb)} "
                    f"code_object={code_object_hash(k) or '-'}")
    lines += ["#", "# machine-readable (bench.py: roofline.traffic = read + write bytes per dispatch)"] + mach
    open(out, "w").write("\n".join(lines) + "\n")


def derived(med):
    """Busy fractions from one run's medians (rocprofv3's derived-metric
    formulas; GRBM_GUI_ACTIVE is summed over the XCDs in these CSVs, so its
    per-XCD value, the kernel's cycles, is the sum / XCDS):
      valu_busy  = SQ_ACTIVE_INST_VALU / (CUS * cycles)      (rocprofv3 VALUBusy / 100)
      lds_busy   = SQ_ACTIVE_INST_LDS / (CUS * cycles)       (the same formula for the LDS)
      lds_bank_conflict = SQ_LDS_BANK_CONFLICT / (CUS * cycles)  (rocprofv3 LDSBankConflict / 100)
      mfma_busy  = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDS * cycles)
      mfma_coexec = SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES (MFMA time with VALU issuing beside it)
      ta_stalled_by_tc = TA_ADDR_STALLED_BY_TC_CYCLES / TA_TA_BUSY (share of the address unit's busy time
                   spent waiting for the L1)"""
    out = {}
    g = med.get("GRBM_GUI_ACTIVE")
    if g:
        cyc = g / XCDS
        if "SQ_ACTIVE_INST_VALU" in med:
            out["valu_busy"] = med["SQ_ACTIVE_INST_VALU"] / (CUS * cyc)
        if "SQ_ACTIVE_INST_LDS" in med:
            out["lds_busy"] = med["SQ_ACTIVE_INST_LDS"] / (CUS * cyc)
        if "SQ_LDS_BANK_CONFLICT" in med:
            out["lds_bank_conflict"] = med["SQ_LDS_BANK_CONFLICT"] / (CUS * cyc)
        if "SQ_VALU_MFMA_BUSY_CYCLES" in med:
            out["mfma_busy"] = med["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMDS * cyc)
    if med.get("SQ_VALU_MFMA_BUSY_CYCLES") and "SQ_VALU_MFMA_COEXEC_CYCLES" in med:
        out["mfma_coexec"] = med["SQ_VALU_MFMA_COEXEC_CYCLES"] / med["SQ_VALU_MFMA_BUSY_CYCLES"]
    if med.get("TA_TA_BUSY") and "TA_ADDR_STALLED_BY_TC_CYCLES" in med:
        out["ta_stalled_by_tc"] = med["TA_ADDR_STALLED_BY_TC_CYCLES"] / med["TA_TA_BUSY"]
    return out


def counters(out, dirs, title, cmd):
    lines = _header(title, cmd)
    lines.append("# medians over the dispatches of each kernel; counters summed over their hardware instances")
    for d in dirs:
        for k, cs in sorted(_counters(d).items()):
            if not k.startswith("dsmoe_") or k == "dsmoe_synth":
                continue
            med = {c: statistics.median(v) for c, v in cs.items()}
            vals = "  ".join(f"{c}={m:.4g}" for c, m in sorted(med.items()))
            vals += "".join(f"  {n}={v:.3f}" for n, v in derived(med).items())
            lines.append(f"{k}  code_object={code_object_hash(k) or '-'}  {vals}")
    open(out, "w").write("\n".join(lines) + "\n")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["kernels", "traffic", "counters"])
    ap.add_argument("out")
    ap.add_argument("dirs", nargs="+")
    ap.add_argument("--title", default="")
    ap.add_argument("--cmd", default="")
    ap.add_argument("--config", default="")
    ap.add_argument("--path", default="")
    a = ap.parse_args()
    if a.mode == "kernels":
        kernels(a.out, a.dirs[0], a.title, a.cmd)
    elif a.mode == "traffic":
        traffic(a.out, a.dirs[0], a.dirs[1], a.config, a.path, a.title, a.cmd)
    else:
        counters(a.out, a.dirs, a.title, a.cmd)


if __name__ == "__main__":
    main()
