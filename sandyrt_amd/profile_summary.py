"""Turn rocprofv3 output of bench.py runs into the tables under profiles/.

    python -m sandyrt_amd.profile_summary trace <kernel_trace.csv> [...]
    python -m sandyrt_amd.profile_summary traffic <fetch counter_collection.csv> <write counter_collection.csv>
    python -m sandyrt_amd.profile_summary traffic_bench <fetch csv> <write csv> <bench.py output of the fetch run>
    python -m sandyrt_amd.profile_summary mfma <counter_collection.csv>
    python -m sandyrt_amd.profile_summary bench_rows <saved traffic table> <bench.py output of the fetch run>

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
            if "at::" in name or "distribution_" in name or name.startswith("__amd_rocclr"):  # input setup copies/fills
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


def _largest(path, counter):
    """The largest single-dispatch value of `counter` among sandy_ew dispatches."""
    vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path))
            if _short(r["Kernel_Name"]) == "sandy_ew" and r["Counter_Name"] == counter]
    return max(vals) if vals else None


def traffic(fetch_path, write_path, copy_bytes=256 << 20):
    """HBM bytes per dispatch: FETCH_SIZE and WRITE_SIZE (KiB), each scaled by
    what it reads for the identity copy of `copy_bytes` that bench.py
    --calibrate-copy runs (the largest sandy_ew dispatch; other generated
    groups can share its grid, so the dispatch is picked by its counter).
    The calibration copy's own grid row and the framework's input-setup
    kernels are left out of the table."""
    f, w = _counters(fetch_path), _counters(write_path)
    fmax, wmax = _largest(fetch_path, "FETCH_SIZE"), _largest(write_path, "WRITE_SIZE")
    rs = copy_bytes / (fmax * 1024) if fmax else 1.0
    ws = copy_bytes / (wmax * 1024) if wmax else 1.0
    out = [f"Scale factors from the {copy_bytes >> 20} MiB identity copy: read {rs:.4f}, write {ws:.4f}.", "",
           "| rocprof kernel | grid | FETCH KiB | WRITE KiB | traffic bytes |", "|---|---|---|---|---|"]
    for key in sorted(f, key=lambda k: k[0]):
        if key[0].startswith(("at::", "__amd_", "(anonymous")) or "FETCH_SIZE" not in f[key] or "WRITE_SIZE" not in w.get(key, {}):
            continue
        if key[0] == "sandy_ew" and fmax and max(f[key]["FETCH_SIZE"]) == fmax:
            # the calibration copy's grid: keep the other groups' dispatches only
            f[key]["FETCH_SIZE"] = [v for v in f[key]["FETCH_SIZE"] if v < 0.5 * fmax]
            w[key]["WRITE_SIZE"] = [v for v in w[key]["WRITE_SIZE"] if v < 0.5 * wmax]
            if not f[key]["FETCH_SIZE"] or not w[key]["WRITE_SIZE"]:
                continue
        fk = sum(f[key]["FETCH_SIZE"]) / len(f[key]["FETCH_SIZE"])
        wk = sum(w[key]["WRITE_SIZE"]) / len(w[key]["WRITE_SIZE"])
        out.append(f"| `{key[0]}` | {key[1]} | {fk:.0f} | {wk:.0f} | {fk * 1024 * rs + wk * 1024 * ws:.0f} |")
    return "\n".join(out)


# bench.py kernel name -> (rocprof kernel name, grid in threads) of its dispatch
# in a `bench.py --no-decode-step` run (config 2/3 step kernels and extras)
BENCH_DISPATCH = {
    "add_rms_norm": ("rms_rows_kernel<sandy_hip::BF16, 4, true, true, true, false>", "262144"),
    "rope_qk": ("rope_split_lines_kernel<sandy_hip::BF16, 6, true, false>", "196608"),
    "silu_gate": ("sandy_ew", "524288"),
    "paged_decode": ("paged_decode_units_kernel<64, 2, 8, 2, 1>", "262144"),
    "c4_paged_decode": ("paged_decode_units_kernel<256, 1, 8, 2, 2>", "524288"),
    "c4_rms_norm": ("rms_rows_kernel<sandy_hip::BF16, 8, false, true, false, true>", "4096"),
    "c4_geglu": ("sandy_ew", "40960"),
    "c4_greedy_argmax": ("argmax_wide_kernel<sandy_hip::BF16, 4, true>", "524288"),
    "c1_greedy_argmax": ("argmax_wide_kernel<sandy_hip::F32, 2, false>", "3328"),
    "c3_qkv_proj": ("sandy_hip::gemm_waves_kernel<1, 2, 4, 8, 1, false, false>", "40960"),
    "c3_o_proj": ("sandy_hip::gemm_waves_kernel<1, 1, 4, 8, 1, false, false>", "65536"),
    "c3_gate_up_proj": ("sandy_hip::gemm_waves_kernel<1, 2, 2, 8, 4, false, false>", "180224"),
    "c3_down_proj": ("sandy_hip::gemm_waves_kernel<1, 2, 2, 8, 4, false, false>", "98304"),
    "c3_lm_head": ("sandy_hip::gemm_waves_kernel<2, 4, 2, 8, 2, false, false>", "128000"),
    "c2_rope_qk_cached": ("rope_split_lines_kernel<sandy_hip::BF16, 6, true, true>", "196608"),
    "c2_rope_cache": ("rope_cache_kernel", "131072"),
    "c2_copy_rope_bytes": ("layout_copy16_kernel", "1179648"),
    "c5_topk": ("topk_rank4_kernel<sandy_hip::F32, 2>", "131072"),
    "c5_moe_gather": ("moe_dispatch_tokens_kernel<16, 8, true>", "65536"),
    "c5_moe_matmul_gate": ("moe_gemm_lines_kernel<4, 4>", "98304"),
    "c5_swiglu": ("sandy_ew", "180224"),
    "c5_moe_matmul_down": ("moe_gemm_lines_kernel<4, 4>", "360448"),
    "c5_moe_scatter_sum": ("moe_combine_kernel<sandy_hip::BF16>", "196608"),
}


def traffic_bench(fetch_path, write_path, bench_log):
    """The traffic table (traffic()) followed by its rows for the bench
    kernels against their algorithmic bytes (the JSON line of `bench_log`)."""
    return bench_rows(traffic(fetch_path, write_path), bench_log)


def bench_rows(table, bench_log):
    """A traffic() table followed by its rows for the bench kernels (also
    usable on a table saved earlier: `bench_rows <table.md> <bench log>`)."""
    import json
    rows = {}
    for line in table.splitlines():
        cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[4].isdigit():
            rows[(cells[0], cells[1])] = (cells[2], cells[3], int(cells[4]))
    line = next(l for l in open(bench_log) if l.startswith("{"))
    d = json.loads(line)
    algo = {k: v["bytes"] for k, v in {**d.get("kernels", {}), **d.get("extras", {})}.items()}
    out = [table, "", "| bench kernel | rocprof kernel (grid) | FETCH KiB | WRITE KiB | traffic bytes | algorithmic bytes | "
           "traffic / algorithmic |", "|---|---|---|---|---|---|---|"]
    for name, (kern, grid) in BENCH_DISPATCH.items():
        if (kern, grid) in rows and name in algo:
            fk, wk, tb = rows[(kern, grid)]
            out.append(f"| {name} | `{kern}` ({grid}) | {fk} | {wk} | {tb} | {algo[name]} | {tb / algo[name]:.3f} |")
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


def _table_of(path):
    """The first markdown table (and the line above it) of a saved traffic table."""
    lines = open(path).read().splitlines()
    out, seen = [], False
    for line in lines:
        if line.startswith("|"):
            seen = True
            out.append(line)
        elif seen:
            break
    return "\n".join(out)


def main(argv):
    if len(argv) < 2:
        print(__doc__)
        return 2
    kind, args = argv[0], argv[1:]
    print(f"source stamp: `{source_stamp()}`\n")
    print({"trace": lambda: trace(args), "traffic": lambda: traffic(*args[:2]),
           "traffic_bench": lambda: traffic_bench(*args[:3]), "mfma": lambda: mfma(args[0]),
           "bench_rows": lambda: bench_rows(_table_of(args[0]), args[1])}[kind]())
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
