"""Per-op SQ counters from one rocprofv3 counter pass, for the ops the
bench runs alone (``bench.py --traffic-runs R --traffic-ops LABELS``: a
1 GiB device-to-device copy, then the op alone R times, per op).

    rocprofv3 --kernel-trace --pmc SQ_INSTS_VALU SQ_INSTS_MFMA \\
        SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_WAVES \\
        SQ_INSTS_LDS SQ_INSTS_SALU GRBM_GUI_ACTIVE -d <dir> -o p \\
        --output-format csv -- python3 bench.py --traffic-runs R \\
        --traffic-ops LABELS > <log>
    python -m dgen_hip.counters <log> <dir> --md <summary.md>

Each counter is the dispatch's total over the chip.  Derived, per op run:
- the shader clock: GRBM_GUI_ACTIVE / 8 (one count per XCD) / duration;
- matrix-core busy: SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x elapsed
  cycles); SQ_VALU_MFMA_BUSY_CYCLES / SQ_INSTS_MFMA is 32 for the
  32x32x16 bf16 MFMA, the cycles one takes on its SIMD, which checks the
  normalisation;
- VALU issue: SQ_INSTS_VALU x 4 cycles (a wave64 VALU instruction holds its
  SIMD four cycles) / (1024 x elapsed cycles).
For dispatches shorter than ~60 us GRBM_GUI_ACTIVE reads more cycles than
the dispatch can hold (the derived clock comes out above the part's 2.4 GHz
peak), so the fractions against it are low there; the columns priced at
the 2.4 GHz peak clock are lower bounds for every op.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os

SIMDS = 1024
XCDS = 8
PEAK_GHZ = 2.4


def _dispatches(directory: str):
    """Dispatch id -> {name, ns, counters...} in dispatch order."""
    d = collections.OrderedDict()
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as fh:
            for r in csv.DictReader(fh):
                e = d.setdefault(int(r["Dispatch_Id"]), {
                    "name": r["Kernel_Name"],
                    "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
                e[r["Counter_Name"]] = float(r["Counter_Value"])
    return [d[k] for k in sorted(d)]


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "").replace("dgen::", "")
    name = name[5:] if name.startswith("void ") else name
    return name.split("(")[0]


def measure(log_path: str, directory: str) -> dict:
    with open(log_path) as fh:
        info = json.loads([ln for ln in fh if ln.startswith("{")][-1])
    ops, runs = info["traffic_ops"], info["runs"]
    rows = _dispatches(directory)
    copies = [i for i, e in enumerate(rows) if "copyBuffer" in e["name"]]
    big = max(rows[i].get("SQ_WAVES", 0.0) for i in copies)
    seps = [i for i in copies if rows[i].get("SQ_WAVES", 0.0) > 0.25 * big][-len(ops):]
    if len(seps) != len(ops):
        raise SystemExit(f"expected {len(ops)} copy separators, found {len(seps)}")
    out = {}
    for k, label in enumerate(ops):
        stop = seps[k + 1] if k + 1 < len(seps) else len(rows)
        grp = [e for e in rows[seps[k] + 1:stop] if not e["name"].startswith("__amd_rocclr")]
        keys = [c for c in grp[0] if c not in ("name", "ns")]
        tot = {c: sum(e.get(c, 0.0) for e in grp) / runs for c in keys}
        ns = sum(e["ns"] for e in grp) / runs
        grbm = tot.get("GRBM_GUI_ACTIVE", 0.0)
        cyc = grbm / XCDS  # elapsed cycles (per XCD)
        r = {"kernels": sorted({_short(e["name"]) for e in grp}), "dispatches_per_run": len(grp) / runs,
             "us": ns / 1e3, "clock_ghz": cyc / ns if ns else 0.0, "counters": tot}
        if cyc > 0:
            r["mfma_busy"] = tot.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (SIMDS * cyc)
            r["valu_issue"] = 4.0 * tot.get("SQ_INSTS_VALU", 0.0) / (SIMDS * cyc)
        if ns:
            r["mfma_busy_peak_clock"] = tot.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (SIMDS * ns * PEAK_GHZ)
            r["valu_issue_peak_clock"] = 4.0 * tot.get("SQ_INSTS_VALU", 0.0) / (SIMDS * ns * PEAK_GHZ)
        if tot.get("SQ_INSTS_MFMA"):
            r["cycles_per_mfma"] = tot["SQ_VALU_MFMA_BUSY_CYCLES"] / tot["SQ_INSTS_MFMA"]
        if tot.get("SQ_WAVES"):
            r["valu_per_wave"] = tot.get("SQ_INSTS_VALU", 0.0) / tot["SQ_WAVES"]
        out[label] = r
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("log")
    ap.add_argument("dir")
    ap.add_argument("--md", required=True)
    args = ap.parse_args()
    res = measure(args.log, args.dir)
    lines = ["| Op | Kernels | µs alone | clock GHz (GRBM) | MFMA busy (GRBM cycles / at 2.4 GHz) | "
             "VALU issue (GRBM cycles / at 2.4 GHz) | VALU instr / wave | MFMA busy cycles / MFMA |",
             "|---|---|---:|---:|---:|---:|---:|---:|"]
    for label, r in res.items():
        cpm = r.get("cycles_per_mfma")
        lines.append(f"| {label} | {', '.join('`' + k + '`' for k in r['kernels'])} | {r['us']:.1f} | "
                     f"{r['clock_ghz']:.2f} | {100 * r.get('mfma_busy', 0.0):.0f}% / "
                     f"{100 * r.get('mfma_busy_peak_clock', 0.0):.0f}% | {100 * r.get('valu_issue', 0.0):.0f}% / "
                     f"{100 * r.get('valu_issue_peak_clock', 0.0):.0f}% | {r.get('valu_per_wave', 0.0):.0f} | "
                     f"{'—' if cpm is None else f'{cpm:.1f}'} |")
    text = "\n".join(lines) + "\n"
    with open(args.md, "w") as fh:
        fh.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
