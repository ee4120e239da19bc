"""HBM traffic of one schedule op, from two rocprofv3 counter passes.

The driver (``bench.py --workload W --traffic-runs R``) sets the session up,
then for each measured op runs a plain 1 GiB device-to-device copy (the HIP
runtime's ``copyBuffer`` kernel, the calibration: it reads and writes
``COPY_BYTES``) followed by the op alone, ``R`` times (``dgen_hip_run_op``),
and prints one JSON line naming the ops.  Under

    rocprofv3 --pmc FETCH_SIZE -d <fetch_dir> -o p --output-format csv -- \
        python3 bench.py --workload W --traffic-runs R > <log>
    rocprofv3 --pmc WRITE_SIZE -d <write_dir> -o p --output-format csv -- \
        python3 bench.py --workload W --traffic-runs R

every dispatch gets its counter in KiB.  Each counter is scaled by what it
reads for the copy (``COPY_BYTES`` / reading): on gfx950 FETCH_SIZE reads
about half of the bytes a plain copy fetches, WRITE_SIZE reads them in full.
The dispatches between one copy and the next are the op's ``R`` runs:

    traffic = sum(FETCH * f_read + WRITE * f_write) / R   bytes per run

``python -m dgen_hip.traffic W <log> <fetch_dir> <write_dir> --json F
--md M`` merges the result into ``F`` (read by bench.py for the
``roofline.traffic`` field) and writes the summary ``M``.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os

COPY_BYTES = 1 << 30


def _dispatches(directory: str) -> list[tuple[int, str, float]]:
    """(dispatch id, kernel name, counter value) in dispatch order."""
    rows = []
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as fh:
            for r in csv.DictReader(fh):
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def _short(name: str) -> str:
    """Kernel name without namespaces, return type and argument list."""
    name = name.replace("(anonymous namespace)::", "").replace("dgen::", "")
    name = name[5:] if name.startswith("void ") else name
    return name.split("(")[0]


def _is_copy(name: str) -> bool:
    return "copyBuffer" in name


def _groups(rows):
    """Split the dispatches after the first large copy into
    (copy reading, [op dispatches]); earlier copies are the setup's uploads."""
    big = max(v for _, n, v in rows if _is_copy(n))
    groups, cur = [], None
    for _, name, v in rows:
        if _is_copy(name) and v > 0.25 * big:
            cur = (v, [])
            groups.append(cur)
        elif cur is not None and not name.startswith("__amd_rocclr"):
            cur[1].append((name, v))
    return groups


def measure(log_path: str, fetch_dir: str, write_dir: str) -> dict:
    with open(log_path) as fh:
        info = json.loads([ln for ln in fh if ln.startswith("{")][-1])
    ops, runs = info["traffic_ops"], info["runs"]
    gf, gw = _groups(_dispatches(fetch_dir)), _groups(_dispatches(write_dir))
    if len(gf) != len(ops) or len(gw) != len(ops):
        raise SystemExit(f"expected {len(ops)} copy-separated groups, found {len(gf)} / {len(gw)}")
    out = {}
    for label, (cf, df), (cw, dw) in zip(ops, gf, gw):
        f_read = COPY_BYTES / (cf * 1024.0)
        f_write = COPY_BYTES / (cw * 1024.0)
        fetch = sum(v for _, v in df) * 1024.0 * f_read / runs
        write = sum(v for _, v in dw) * 1024.0 * f_write / runs
        kernels = sorted({_short(n) for n, _ in df})
        out[label] = {"bytes_per_run": fetch + write, "fetch_bytes": fetch, "write_bytes": write,
                      "read_factor": f_read, "write_factor": f_write, "runs": runs,
                      "dispatches_per_run": len(df) / runs, "kernels": kernels}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("workload")
    ap.add_argument("log")
    ap.add_argument("fetch_dir")
    ap.add_argument("write_dir")
    ap.add_argument("--json", required=True)
    ap.add_argument("--md", required=True)
    args = ap.parse_args()
    res = measure(args.log, args.fetch_dir, args.write_dir)
    runs = next(iter(res.values()))["runs"]
    data = {}
    if os.path.exists(args.json):
        with open(args.json) as fh:
            data = json.load(fh)
    data[args.workload] = res
    with open(args.json, "w") as fh:
        json.dump(data, fh, indent=1, sort_keys=True)
        fh.write("\n")
    lines = [f"# HBM traffic per op run: {args.workload}", "",
             "Commands (repository root, one MI355X, `TMPDIR=/tmp`):", "", "```",
             f"rocprofv3 --pmc FETCH_SIZE -d <fetch_dir> -o p --output-format csv -- python3 bench.py "
             f"--workload {args.workload} --traffic-runs {runs} > <log>",
             f"rocprofv3 --pmc WRITE_SIZE -d <write_dir> -o p --output-format csv -- python3 bench.py "
             f"--workload {args.workload} --traffic-runs {runs}",
             f"python -m dgen_hip.traffic {args.workload} <log> <fetch_dir> <write_dir> --json ... --md ...", "```",
             "", "Counters scaled by a 1 GiB device-to-device copy measured in the same run "
             "(bytes copied / counter reading).",
             "", "| Op | Kernels | Dispatches/run | Read MB/run | Write MB/run | Total MB/run | "
             "Read factor | Write factor |", "|---|---|---:|---:|---:|---:|---:|---:|"]
    for label, r in res.items():
        lines.append(f"| {label} | {', '.join('`' + k + '`' for k in r['kernels'])} | {r['dispatches_per_run']:.0f} | "
                     f"{r['fetch_bytes'] / 1e6:.2f} | {r['write_bytes'] / 1e6:.2f} | {r['bytes_per_run'] / 1e6:.2f} | "
                     f"{r['read_factor']:.3f} | {r['write_factor']:.3f} |")
    with open(args.md, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
