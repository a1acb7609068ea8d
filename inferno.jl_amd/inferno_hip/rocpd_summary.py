"""Summarize a rocprofv3 result database (rocpd SQLite) as a Markdown table.

    python -m inferno_hip.rocpd_summary trace_results.db            # kernel trace
    python -m inferno_hip.rocpd_summary fetch_results.db --pmc      # counters
    python -m inferno_hip.rocpd_summary fetch.db --traffic write.db # HBM bytes

Kernel trace: per kernel, dispatches and duration statistics (ns).  Counters:
per kernel and counter, dispatches and the mean / min / max value per
dispatch.  Traffic: a FETCH_SIZE and a WRITE_SIZE run of the same program
(bench.py --pmc-workload), each counter scaled by what it reads for the
program's 64 MiB device-to-device copies (the copy kernels whose WRITE_SIZE is
65536 KiB), then HBM bytes per dispatch per kernel.  Kernel names are
demangled and shortened to the template head (`ihip::` and argument lists
dropped).  This is how the summaries under profiles/ are made
from the databases rocprofv3 writes.
"""
from __future__ import annotations

import argparse
import re
import sqlite3
import statistics
import subprocess
from collections import defaultdict


def demangle(name: str) -> str:
    if not name.startswith("_Z"):
        return name
    try:
        r = subprocess.run(["c++filt", name], capture_output=True, text=True, check=True)
        if r.stdout.strip() and r.stdout.strip() != name:
            return r.stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        pass
    # c++filt does not know every type (e.g. _Float16): keep the nested name
    # and the literal template arguments (bool / int) of its components
    if not name.startswith("_ZN"):
        return name
    parts, rest = [], name[3:]
    while rest and rest[0].isdigit():
        k = re.match(r"(\d+)", rest)
        s, n = len(k.group(1)), int(k.group(1))
        parts.append(rest[s:s + n])
        rest = rest[s + n:]
        if rest.startswith("I"):
            args, rest = [], rest[1:]
            while rest and rest[0] != "E":
                a = re.match(r"L([bij])(n?\d+)E", rest)
                if not a:
                    return "::".join(parts) + "<...>"
                v = a.group(2).replace("n", "-")
                args.append(("true" if v == "1" else "false") if a.group(1) == "b" else v)
                rest = rest[a.end():]
            rest = rest[1:]
            parts[-1] += "<" + ", ".join(args) + ">"
    return "::".join(parts) if parts else name


def short(name: str, width: int = 90) -> str:
    n = demangle(name.strip()).replace("(anonymous namespace)::", "")
    n = re.sub(r"\(.*\)$", "", n)
    n = n.replace("void ", "").replace("ihip::", "")
    return n if len(n) <= width else n[: width - 3] + "..."


def kernel_rows(db: str):
    cur = sqlite3.connect(db).cursor()
    rows = cur.execute("select name, duration from kernels").fetchall()
    by = defaultdict(list)
    for name, d in rows:
        by[name].append(int(d))
    out = []
    for name, ds in by.items():
        out.append((short(name), len(ds), statistics.mean(ds), statistics.median(ds), min(ds), max(ds),
                    sum(ds)))
    out.sort(key=lambda r: -r[6])
    return out


def pmc_rows(db: str):
    cur = sqlite3.connect(db).cursor()
    rows = cur.execute("select kernel_name, counter_name, value from counters_collection").fetchall()
    by = defaultdict(list)
    for k, c, v in rows:
        by[(k, c)].append(float(v))
    out = [(short(k), c, len(vs), statistics.mean(vs), min(vs), max(vs)) for (k, c), vs in by.items()]
    out.sort(key=lambda r: (r[1], r[0]))
    return out


def traffic_rows(fetch_db: str, write_db: str):
    """(fetch factor, write factor, rows of (kernel, dispatches, fetched bytes,
    written bytes) per dispatch), dispatches matched by their order."""
    def per_dispatch(db, ctr):
        cur = sqlite3.connect(db).cursor()
        return cur.execute("select dispatch_id, kernel_name, value from counters_collection "
                           "where counter_name = ? order by dispatch_id", (ctr,)).fetchall()
    f, w = per_dispatch(fetch_db, "FETCH_SIZE"), per_dispatch(write_db, "WRITE_SIZE")
    if len(f) != len(w) or any(a[1] != b[1] for a, b in zip(f, w)):
        raise SystemExit("the two runs dispatched different kernels")
    cal = [(a[2], b[2]) for a, b in zip(f, w) if "copyBuffer" in a[1] and abs(b[2] - 65536.0) < 1]
    if not cal:
        raise SystemExit("no 64 MiB copy to calibrate against")
    ff = 65536.0 / statistics.mean(c[0] for c in cal)
    wf = 65536.0 / statistics.mean(c[1] for c in cal)
    by = defaultdict(list)
    for a, b in zip(f, w):
        by[a[1]].append((a[2] * ff * 1024, b[2] * wf * 1024))
    out = [(short(k), len(v), statistics.mean(x[0] for x in v), statistics.mean(x[1] for x in v))
           for k, v in by.items()]
    out.sort(key=lambda r: -(r[2] + r[3]))
    return ff, wf, out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("--pmc", action="store_true")
    ap.add_argument("--traffic", metavar="WRITE_DB", help="db is the FETCH_SIZE run; this the WRITE_SIZE run")
    ap.add_argument("--match", default="", help="only kernels whose name contains this")
    a = ap.parse_args()
    if a.traffic:
        ff, wf, rows = traffic_rows(a.db, a.traffic)
        print(f"FETCH_SIZE x {ff:.5f}, WRITE_SIZE x {wf:.5f} (64 MiB device copies)\n")
        print("| kernel | dispatches | HBM read B | HBM write B |")
        print("|---|---|---|---|")
        for k, n, rd, wr in rows:
            if a.match in k:
                print(f"| `{k}` | {n} | {rd:,.0f} | {wr:,.0f} |")
    elif a.pmc:
        print("| kernel | counter | dispatches | mean | min | max |")
        print("|---|---|---|---|---|---|")
        for k, c, n, mean, lo, hi in pmc_rows(a.db):
            if a.match in k:
                print(f"| `{k}` | {c} | {n} | {mean:.1f} | {lo:.1f} | {hi:.1f} |")
    else:
        print("| kernel | dispatches | mean ns | median ns | min ns | max ns | total ms |")
        print("|---|---|---|---|---|---|---|")
        for k, n, mean, med, lo, hi, tot in kernel_rows(a.db):
            if a.match in k:
                print(f"| `{k}` | {n} | {mean:.0f} | {med:.0f} | {lo} | {hi} | {tot / 1e6:.3f} |")


if __name__ == "__main__":
    main()
