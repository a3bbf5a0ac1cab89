"""HBM traffic of one kernel from two rocprofv3 --pmc runs, stamped with the kernel's sources.

    python -m cortexsdr_amd.traffic --fetch F.csv --write W.csv --kernel gatherw_kernel \
        --alg-bytes N --out profiles/hsdb_gather_cfg2_traffic.json [--command ...]

F.csv / W.csv are the `run_counter_collection.csv` files of a FETCH_SIZE run and a WRITE_SIZE
run of the same program (KiB per dispatch). Both runs must also hold a plain device copy of
known size (bench.py --calibrate-copy: 256 MiB through `__amd_rocclr_copyBuffer`), whose
counter readings give the scale from counter KiB to bytes moved:

    traffic = (fetch_kib / fetch_scale + write_kib / write_scale) * 1024

The JSON records the digest of the sources the kernel is built from (`source_digest`), so a
reader can tell whether the measurement is of the kernel in the tree: bench.py reports the
traffic only when the digest matches the current sources.
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import os
import statistics
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

# Sources the HSDB product kernels are compiled from (kernels, layout helpers, shared device
# helpers). Any edit to them invalidates a committed traffic measurement.
HSDB_SOURCES = ("csrc/hsdb.hip", "csrc/hsdb_impl.hpp", "csrc/common.hpp")

CALIB_KERNEL = "__amd_rocclr_copyBuffer"
CALIB_BYTES = 256 * 1024 * 1024


def source_digest(paths=HSDB_SOURCES) -> str:
    """First 16 hex digits of the SHA-256 over the named package sources, in order."""
    h = hashlib.sha256()
    for rel in paths:
        with open(os.path.join(HERE, rel), "rb") as f:
            data = f.read()
        h.update(rel.encode() + b"\0" + len(data).to_bytes(8, "little") + data)
    return h.hexdigest()[:16]


def git_head() -> str | None:
    try:
        r = subprocess.run(["git", "-C", ROOT, "rev-parse", "--short=12", "HEAD"],
                           capture_output=True, text=True, timeout=10)
        return r.stdout.strip() or None
    except (OSError, subprocess.SubprocessError):
        return None


def _readings(path: str, counter: str):
    """{kernel name: [values]} for one counter, and the calibration copy's readings."""
    per, calib = {}, []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            v = float(r["Counter_Value"])
            name = r["Kernel_Name"]
            # the calibration copy, not the small staging copies of the same kernel
            if name == CALIB_KERNEL and v >= CALIB_BYTES / 1024 / 4:
                calib.append(v)
            per.setdefault(name, []).append(v)
    return per, calib


def _stats(v):
    return {"mean": round(statistics.fmean(v), 3), "min": min(v), "max": max(v),
            "dispatches": len(v)}


def measure(fetch_csv: str, write_csv: str, kernel: str) -> dict:
    fper, fcal = _readings(fetch_csv, "FETCH_SIZE")
    wper, wcal = _readings(write_csv, "WRITE_SIZE")
    fk = [v for n, vs in fper.items() if kernel in n for v in vs]
    wk = [v for n, vs in wper.items() if kernel in n for v in vs]
    names = sorted({n for n in fper if kernel in n})
    if not fk or not wk:
        raise SystemExit(f"no dispatches of a kernel matching {kernel!r}")
    if not fcal or not wcal:
        raise SystemExit("no calibration copy in the runs (bench.py --calibrate-copy)")
    kib = CALIB_BYTES / 1024
    # the copy reads and writes 256 MiB each
    fs = statistics.median(fcal) / kib
    ws = statistics.median(wcal) / kib
    fm, wm = statistics.fmean(fk), statistics.fmean(wk)
    traffic = (fm / fs + wm / ws) * 1024
    return {
        "kernel_names": names,
        "traffic_bytes": int(round(traffic)),
        "fetch_kib_per_dispatch": _stats(fk),
        "write_kib_per_dispatch": _stats(wk),
        "calibration": {
            "dispatch": f"{CALIB_KERNEL} of 256 MiB (bench.py --calibrate-copy)",
            "fetch_kib": round(statistics.median(fcal), 3),
            "write_kib": round(statistics.median(wcal), 3),
            "bytes_copied_kib": kib,
            "fetch_scale": round(fs, 6),
            "write_scale": round(ws, 6),
        },
        "formula": "traffic = (fetch_kib / fetch_scale + write_kib / write_scale) * 1024",
    }


def load_current(path: str):
    """The committed measurement if it was made from the current sources, else None; and the
    reason when it is not usable."""
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, "missing"
    want = source_digest(tuple(t.get("sources", HSDB_SOURCES)))
    if t.get("source_digest") != want:
        return None, f"stale (measured at sources {t.get('source_digest')}, tree {want})"
    return t, None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--kernel", required=True, help="substring of the kernel name")
    ap.add_argument("--label", default=None, help="kernel and workload described")
    ap.add_argument("--alg-bytes", type=int, required=True)
    ap.add_argument("--out", required=True)
    ap.add_argument("--command", action="append", default=[],
                    help="the rocprofv3 commands that produced the CSVs (repeatable)")
    a = ap.parse_args(argv)
    m = measure(a.fetch, a.write, a.kernel)
    out = {
        "kernel": a.label or a.kernel,
        **m,
        "algorithmic_bytes": a.alg_bytes,
        "traffic_over_algorithmic": round(m["traffic_bytes"] / a.alg_bytes, 4),
        "sources": list(HSDB_SOURCES),
        "source_digest": source_digest(),
        "git_head": git_head(),
        "commands": a.command,
        "device": "MI355X (gfx950), one GPU",
    }
    with open(a.out, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps({k: out[k] for k in ("traffic_bytes", "traffic_over_algorithmic",
                                          "source_digest", "git_head")}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
