"""Summaries of rocprofv3 output for profiles/ (host only, no GPU).

Two kinds, both stamped with the SHA-256 prefix of the library the profiled run loaded (`lib_sha16`, printed by
bench.py in its JSON line), so bench.py can refuse figures that belong to another build:

* kernel trace (`rocprofv3 --kernel-trace --stats --output-format csv -d DIR -o run -- python3 bench.py ...`):
  `profiles/<kernel>_<workload>.md` (top kernels by total time, the bench line of the same run) and
  `profiles/trace_<key>_<workload>.json` (per-dispatch durations of the named kernel: all dispatches and the last
  `--last` ones, i.e. the timed steps);
* HBM traffic from two counter runs (`rocprofv3 --pmc FETCH_SIZE ...`, then `--pmc WRITE_SIZE ...`, each with
  bench.py --copy-probe): `profiles/traffic_<key>_<workload>.json`. FETCH_SIZE and WRITE_SIZE are in KiB per dispatch;
  each is scaled by what the same counter reads for the probe's plain 1 GiB device copy (1 GiB read + 1 GiB written).

* matrix-core, LDS and VALU counters (`rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16
  SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_VALU SQ_BUSY_CU_CYCLES SQ_INSTS_LDS
  GRBM_GUI_ACTIVE ...`, one run per workload): a markdown table `profiles/<out>.md`, one row per (workload, kernel).

usage:
  python -m loki_amd.profsum counters --out NAME --cmd "..." --last N WORKLOAD=DIR=LOG ... --kernels REGEX ...
  python -m loki_amd.profsum trace DIR --kernel REGEX --key KEY --workload W --last N --log BENCH_STDOUT --cmd "..." [--group G]
  python -m loki_amd.profsum traffic FETCH_DIR WRITE_DIR --kernel REGEX --key KEY --workload W --last N
         --alg BYTES --log-fetch LOG --log-write LOG --cmd-fetch "..." --cmd-write "..." [--notes "..."] [--group G]
(--group G: a stage launched as G kernels back to back, their consecutive dispatches summed per step)
"""
import argparse
import csv
import glob
import json
import os
import re
import statistics

HERE = os.path.dirname(os.path.abspath(__file__))
PROFILES = os.path.join(os.path.dirname(HERE), "profiles")
GiB = 1 << 30


def _find(d, suffix):
    f = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not f:
        raise SystemExit("no *%s under %s" % (suffix, d))
    return f[-1]


def _short(name):
    n = name.replace("(anonymous namespace)::", "")
    m = re.match(r"^(void )?([^()]*?)(\(.*)?$", n)
    return (m.group(2) if m else n).strip()[:60]


def bench_line(log_path):
    """The last JSON object printed by bench.py in a log (stdout + stderr), or None."""
    last = None
    with open(log_path, errors="replace") as f:
        for line in f:
            s = line.strip()
            if s.startswith("[bench]"):
                continue
            i = s.find("{")
            if i < 0:
                continue
            try:
                obj = json.loads(s[i:])
            except ValueError:
                continue
            if isinstance(obj, dict):
                last = obj
    return last


def lib_of(log_path):
    b = bench_line(log_path)
    if not b or "lib_sha16" not in b:
        raise SystemExit("%s: no bench line with lib_sha16" % log_path)
    return b["lib_sha16"], b


def _durations(trace_csv, pat):
    rx = re.compile(pat)
    out = []
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            if rx.search(r["Kernel_Name"]):
                out.append((int(r["Start_Timestamp"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    out.sort()
    return [d for _, d in out]


def _grouped(d, g):
    """Consecutive dispatches summed in groups of g (a stage launched as g kernels back to back, e.g. the prefill
    GEMM's wide and narrow kernels); trailing partial groups are dropped."""
    if g <= 1:
        return d
    return [sum(d[i:i + g]) for i in range(0, len(d) - len(d) % g, g)]


def trace(a):
    tcsv, scsv = _find(a.dir, "kernel_trace.csv"), _find(a.dir, "kernel_stats.csv")
    sha, line = lib_of(a.log)
    d = _grouped(_durations(tcsv, a.kernel), a.group)
    if not d:
        raise SystemExit("kernel /%s/ not in %s" % (a.kernel, tcsv))
    last = d[-a.last:] if a.last else d
    rows = sorted(csv.DictReader(open(scsv)), key=lambda r: -int(r["TotalDurationNs"]))
    js = {"kernel": a.key, "kernel_regex": a.kernel, "workload": a.workload, "lib_sha16": sha,
          "dispatches": len(d), "avg_us_all": round(sum(d) / len(d), 3),
          "last_n": len(last), "avg_us_last": round(sum(last) / len(last), 3),
          "median_us_last": round(statistics.median(last), 3), "min_us_last": round(min(last), 3),
          "max_us_last": round(max(last), 3), "kernels_per_step": a.group, "command": a.cmd,
          "bench_roofline": line.get("roofline") if line else None,
          "bench_value": line.get("value") if line else None}
    os.makedirs(PROFILES, exist_ok=True)
    with open(os.path.join(PROFILES, "trace_%s_%s.json" % (a.key, a.workload)), "w") as f:
        json.dump(js, f, indent=1)
        f.write("\n")
    md = ["# %s, %s -- rocprofv3 kernel trace" % (a.key, a.workload), "",
          "Library `libloki_moe.so` sha256 prefix `%s` (the bench line's `lib_sha16`)." % sha, "",
          "Command (repo root, on the MI355X box):", "", "    " + a.cmd, "",
          "The named kernel over its last %d dispatches (the timed steps): average %.2f us, median %.2f, min %.2f, max "
          "%.2f (all %d dispatches: average %.2f us)." % (len(last), js["avg_us_last"], js["median_us_last"],
                                                       js["min_us_last"], js["max_us_last"], len(d), js["avg_us_all"]),
          "", "| kernel | calls | avg us | min us | max us | % time |", "|---|---:|---:|---:|---:|---:|"]
    for r in rows[:a.top]:
        md.append("| %s | %s | %.2f | %.2f | %.2f | %s |" % (_short(r["Name"]), r["Calls"], float(r["AverageNs"]) / 1e3,
                                                            int(r["MinNs"]) / 1e3, int(r["MaxNs"]) / 1e3, r["Percentage"]))
    if line:
        keep = {k: line[k] for k in ("value", "unit", "ms_per_step", "roofline", "lib_sha16") if k in line}
        md += ["", "bench.py line of the same run (under the profiler; its main fields):", "", "    " + json.dumps(keep)]
    if a.notes:
        md += ["", a.notes]
    with open(os.path.join(PROFILES, "%s_%s.md" % (a.key, a.workload)), "w") as f:
        f.write("\n".join(md) + "\n")
    print(json.dumps(js, indent=1))


def _counter(d, ctr):
    f = _find(d, "counter_collection.csv")
    return [r for r in csv.DictReader(open(f)) if r["Counter_Name"] == ctr]


def traffic(a):
    sf, bf = lib_of(a.log_fetch)
    sw, bw = lib_of(a.log_write)
    if sf != sw:
        raise SystemExit("the FETCH_SIZE and WRITE_SIZE runs loaded different libraries (%s, %s)" % (sf, sw))
    rx = re.compile(a.kernel)
    fr, wr = _counter(a.fetch_dir, "FETCH_SIZE"), _counter(a.write_dir, "WRITE_SIZE")

    def kv(rs):
        v = [(int(r["Dispatch_Id"]), float(r["Counter_Value"])) for r in rs if rx.search(r["Kernel_Name"])]
        v.sort()
        return _grouped([x for _, x in v], a.group)[-a.last:]

    def probe(rs):
        v = [float(r["Counter_Value"]) for r in rs if "copyBuffer" in r["Kernel_Name"] and int(r["Grid_Size"]) >= 1 << 17]
        if not v:
            raise SystemExit("no copy-probe dispatch (run bench.py with --copy-probe)")
        return max(v)

    fk, wk = kv(fr), kv(wr)
    if not fk or not wk:
        raise SystemExit("kernel /%s/ not in the counter runs" % a.kernel)
    f_mean, w_mean = sum(fk) / len(fk), sum(wk) / len(wk)
    cf, cw = probe(fr), probe(wr)
    fs, ws = round(GiB / 1024 / cf, 3), round(GiB / 1024 / cw, 3)
    rb, wb = f_mean * 1024 * fs, w_mean * 1024 * ws
    out = {"kernel": a.key, "kernel_regex": a.kernel, "workload": a.workload, "lib_sha16": sf,
           "fetch_size_kib_per_dispatch": round(f_mean, 3), "write_size_kib_per_dispatch": round(w_mean, 3),
           "dispatches_averaged": len(fk), "kernels_per_step": a.group,
           "copy_probe": {"bytes_read": GiB, "bytes_written": GiB, "fetch_size_kib": cf, "write_size_kib": cw},
           "fetch_scale": fs, "write_scale": ws, "bytes_per_launch": int(rb + wb), "read_bytes_per_launch": int(rb),
           "write_bytes_per_launch": int(wb), "algorithmic_bytes_per_launch": a.alg,
           "traffic_over_algorithmic": round((rb + wb) / a.alg, 3) if a.alg else None,
           "commands": [a.cmd_fetch, a.cmd_write], "notes": a.notes or ""}
    os.makedirs(PROFILES, exist_ok=True)
    with open(os.path.join(PROFILES, "traffic_%s_%s.json" % (a.key, a.workload)), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out, indent=1))


PMC = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE",
       "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_VALU", "SQ_BUSY_CU_CYCLES", "SQ_INSTS_LDS", "GRBM_GUI_ACTIVE")


def counters(a):
    """Per (workload, kernel): the mean of each counter over the kernel's last N dispatches, then MFMA busy =
    SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs) (GRBM_GUI_ACTIVE is summed over the 8 XCDs),
    bank conflicts per LDS access = SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT), LDS / VALU
    active = SQ_ACTIVE_INST_LDS / SQ_ACTIVE_INST_VALU over SQ_BUSY_CU_CYCLES."""
    md = ["# %s -- rocprofv3 counters" % a.out, "",
          "Command (repo root, on the MI355X box; WL = each workload below, one run each):", "", "    " + a.cmd, ""]
    shas = set()
    table = ["| workload | kernel | dispatches | MFMA busy | MFMA ops (F16 MOPs) | LDS instructions | LDS conflicts / access | "
             "LDS active | VALU active |", "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    for spec in a.runs:
        wl, d, log = spec.split("=")
        shas.add(lib_of(log)[0])
        rows = _counter_rows(d)
        for krx in a.kernels:
            rx = re.compile(krx)
            names = sorted({r["Kernel_Name"] for r in rows if rx.search(r["Kernel_Name"])})
            for name in names:
                per = {}
                for r in rows:
                    if r["Kernel_Name"] == name and r["Counter_Name"] in PMC:
                        per.setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
                ds = [per[k] for k in sorted(per) if len(per[k]) == len(PMC)][-a.last:]
                if not ds:
                    continue
                m = {c: sum(x[c] for x in ds) / len(ds) for c in PMC}
                busy = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (m["GRBM_GUI_ACTIVE"] / 8 * 1024) if m["GRBM_GUI_ACTIVE"] else 0.0
                acc = m["SQ_LDS_IDX_ACTIVE"] - m["SQ_LDS_BANK_CONFLICT"]
                conf = m["SQ_LDS_BANK_CONFLICT"] / acc if acc > 0 else 0.0
                cu = m["SQ_BUSY_CU_CYCLES"] or 1.0
                table.append("| %s | `%s` | %d | %.1f %% | %.0f M | %.1f M | %.3f | %.0f %% | %.0f %% |" % (
                    wl, _short(name), len(ds), 100 * busy, m["SQ_INSTS_VALU_MFMA_MOPS_F16"] / 1e6, m["SQ_INSTS_LDS"] / 1e6,
                    conf, 100 * m["SQ_ACTIVE_INST_LDS"] / cu, 100 * m["SQ_ACTIVE_INST_VALU"] / cu))
    md.insert(1, "Library `libloki_moe.so` sha256 prefix %s (the bench lines' `lib_sha16`)." % ", ".join("`%s`" % s for s in sorted(shas)))
    md.insert(2, "")
    md += table + ["", counters.__doc__.split("\n", 1)[0].strip().replace("Per (workload, kernel): t", "T") + " " +
                   " ".join(l.strip() for l in counters.__doc__.split("\n")[1:]) + " Mean of the last %d dispatches." % a.last]
    if a.notes:
        md += ["", a.notes]
    with open(os.path.join(PROFILES, a.out + ".md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print("\n".join(table))


def _counter_rows(d):
    return list(csv.DictReader(open(_find(d, "counter_collection.csv"))))


def main(argv=None):
    ap = argparse.ArgumentParser(description="rocprofv3 output -> profiles/ summaries")
    sub = ap.add_subparsers(dest="what", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    for k in ("--kernel", "--key", "--workload", "--log", "--cmd"):
        t.add_argument(k, required=True)
    t.add_argument("--last", type=int, default=0)
    t.add_argument("--group", type=int, default=1, help="kernels per step, summed (consecutive dispatches)")
    t.add_argument("--top", type=int, default=12)
    t.add_argument("--notes", default="")
    p = sub.add_parser("traffic")
    p.add_argument("fetch_dir")
    p.add_argument("write_dir")
    for k in ("--kernel", "--key", "--workload", "--log-fetch", "--log-write", "--cmd-fetch", "--cmd-write"):
        p.add_argument(k, required=True)
    p.add_argument("--last", type=int, default=10)
    p.add_argument("--group", type=int, default=1, help="kernels per step, summed (consecutive dispatches)")
    p.add_argument("--alg", type=int, required=True)
    p.add_argument("--notes", default="")
    c = sub.add_parser("counters")
    c.add_argument("runs", nargs="+", help="WORKLOAD=DIR=BENCH_LOG")
    c.add_argument("--kernels", nargs="+", required=True)
    c.add_argument("--out", required=True)
    c.add_argument("--cmd", required=True)
    c.add_argument("--last", type=int, default=3)
    c.add_argument("--notes", default="")
    a = ap.parse_args(argv)
    {"trace": trace, "traffic": traffic, "counters": counters}[a.what](a)


if __name__ == "__main__":
    main()
