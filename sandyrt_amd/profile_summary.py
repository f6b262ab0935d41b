"""Turn rocprofv3 output of bench.py runs into the tables under profiles/.

    python -m sandyrt_amd.profile_summary trace <kernel_trace.csv> [...]
    python -m sandyrt_amd.profile_summary traffic <fetch counter_collection.csv> <write counter_collection.csv>
    python -m sandyrt_amd.profile_summary mfma <counter_collection.csv>

Every table is stamped with the source stamp of the kernels it measured
(`source_stamp()`: a hash of sandyrt_amd/csrc and include/), so bench.py can
tell whether a committed measurement still describes the code it runs.
"""
from __future__ import annotations

import collections
import csv
import hashlib
import os
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)


def source_stamp() -> str:
    """16 hex digits of the SHA-256 of every kernel source and the C ABI header."""
    h = hashlib.sha256()
    files = []
    for d in (os.path.join(PKG, "csrc"), os.path.join(ROOT, "include")):
        for name in sorted(os.listdir(d)):
            if name.endswith((".hip", ".h", ".cpp")):
                files.append(os.path.join(d, name))
    for f in files:
        h.update(os.path.relpath(f, ROOT).encode())
        h.update(open(f, "rb").read())
    return h.hexdigest()[:16]


def stamp_of(path: str) -> str | None:
    """The `source stamp:` recorded in a profiles/ table, or None."""
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.lower().startswith("source stamp:"):
            return line.split(":", 1)[1].strip().split()[0].strip("`")
    return None


def _short(name: str) -> str:
    name = name.replace("sandy_hip::(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    cut = name.find("(")
    return name[:cut] if cut > 0 else name


def trace(paths):
    """Per (kernel, grid) durations (End - Start) from kernel_trace.csv files."""
    rows = collections.defaultdict(list)
    for p in paths:
        for r in csv.DictReader(open(p)):
            name = r["Kernel_Name"]
            if "at::" in name or "distribution_" in name:  # torch's input setup
                continue
            key = (_short(name), r.get("Grid_Size", r.get("Grid_Size_X", "")), r.get("Workgroup_Size", ""))
            rows[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in rows.values()) or 1.0
    out = ["| kernel | grid (threads) | block | calls | avg us | min us | max us | % of listed time |",
           "|---|---|---|---|---|---|---|---|"]
    for (k, g, b), v in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"| `{k}` | {g} | {b} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                   f"{100 * sum(v) / total:.2f} |")
    return "\n".join(out)


def _counters(path):
    """{(kernel, grid): {counter: [per-dispatch values]}} from counter_collection.csv."""
    d = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(path)):
        d[(_short(r["Kernel_Name"]), r["Grid_Size"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return d


def traffic(fetch_path, write_path, copy_bytes=256 << 20):
    """HBM bytes per dispatch: FETCH_SIZE and WRITE_SIZE (KiB), each scaled by
    what it reads for the identity copy of `copy_bytes` that bench.py
    --calibrate-copy runs (the largest sandy_ew dispatch)."""
    f, w = _counters(fetch_path), _counters(write_path)
    cal = max((k for k in f if k[0] == "sandy_ew"), key=lambda k: int(k[1]), default=None)
    rs = ws = 1.0
    if cal and "FETCH_SIZE" in f[cal] and "WRITE_SIZE" in w.get(cal, {}):
        rs = copy_bytes / (sum(f[cal]["FETCH_SIZE"]) / len(f[cal]["FETCH_SIZE"]) * 1024)
        ws = copy_bytes / (sum(w[cal]["WRITE_SIZE"]) / len(w[cal]["WRITE_SIZE"]) * 1024)
    out = [f"Scale factors from the {copy_bytes >> 20} MiB identity copy: read {rs:.4f}, write {ws:.4f}.", "",
           "| rocprof kernel | grid | FETCH KiB | WRITE KiB | traffic bytes |", "|---|---|---|---|---|"]
    for key in sorted(f, key=lambda k: k[0]):
        if key == cal or "FETCH_SIZE" not in f[key] or "WRITE_SIZE" not in w.get(key, {}):
            continue
        fk = sum(f[key]["FETCH_SIZE"]) / len(f[key]["FETCH_SIZE"])
        wk = sum(w[key]["WRITE_SIZE"]) / len(w[key]["WRITE_SIZE"])
        out.append(f"| `{key[0]}` | {key[1]} | {fk:.0f} | {wk:.0f} | {fk * 1024 * rs + wk * 1024 * ws:.0f} |")
    return "\n".join(out)


def mfma(path, simds=1024):
    """MFMA busy share and MFMA math per dispatch.  SQ_VALU_MFMA_BUSY_CYCLES is
    summed over every SIMD; GRBM_GUI_ACTIVE over the 8 XCDs, so one XCD's
    active cycles (the dispatch's wall-clock in shader cycles) are its eighth."""
    d = _counters(path)
    out = ["| kernel | grid | dispatches | active cycles (per XCD) | MFMA busy cycles (all SIMDs) | MFMA busy % of SIMD "
           "time | MFMA MOPS bf16 (x512 flop) | GFLOP per dispatch |", "|---|---|---|---|---|---|---|---|"]
    for key, c in sorted(d.items()):
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in c or "GRBM_GUI_ACTIVE" not in c:
            continue
        busy = sum(c["SQ_VALU_MFMA_BUSY_CYCLES"]) / len(c["SQ_VALU_MFMA_BUSY_CYCLES"])
        active = sum(c["GRBM_GUI_ACTIVE"]) / len(c["GRBM_GUI_ACTIVE"]) / 8
        mops = sum(c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [0])) / max(1, len(c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [0])))
        if busy == 0:
            continue
        out.append(f"| `{key[0]}` | {key[1]} | {len(c['GRBM_GUI_ACTIVE'])} | {active:.0f} | {busy:.0f} | "
                   f"{100 * busy / (active * simds):.2f} | {mops:.0f} | {mops * 512 / 1e9:.3f} |")
    return "\n".join(out)


def main(argv):
    if len(argv) < 2:
        print(__doc__)
        return 2
    kind, args = argv[0], argv[1:]
    print(f"source stamp: `{source_stamp()}`\n")
    print({"trace": lambda: trace(args), "traffic": lambda: traffic(*args[:2]), "mfma": lambda: mfma(args[0])}[kind]())
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
