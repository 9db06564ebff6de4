"""Turns rocprofv3 output of ``bench.py`` into the short text summaries kept with the measurements.

Inputs are rocprofv3 output directories written with ``-o run --output-format csv``:

  --trace DIR   a ``--kernel-trace --stats`` run   (reads run_kernel_stats.csv)
  --fetch DIR   a ``--pmc FETCH_SIZE`` run          (reads run_counter_collection.csv)
  --write DIR   a ``--pmc WRITE_SIZE`` run
  --pmc DIR     any other ``--pmc`` run (repeatable), e.g. matrix-core busy cycles and LDS bank conflicts

HBM traffic per launch is calibrated against the largest ``__amd_rocclr_copyBuffer`` dispatch of the same run,
a device-to-device copy of ``--copy-bytes`` bytes (``bench.py --kernels-only`` issues one of 256 MiB): the copy
reads and writes exactly that many bytes, so ``factor = bytes / counter`` converts each counter to bytes.

Writes a markdown summary (``--md``) and, with ``--json``, the per-launch traffic that ``bench.py`` reports as
``roofline.traffic``.
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import re
from pathlib import Path

COPY_KERNEL = "__amd_rocclr_copyBuffer"


IO_SUFFIX = {"hb::Bf16Io": "_bf16", "hb::F16Io": "_f16"}


def short_name(name: str) -> str:
    """``void hb::dense_attend<hb::Bf16Io, 64, 128>(...)`` -> ``dense_attend_bf16<64,128>`` (the element type of
    the kernel's inputs becomes a suffix; also through nested namespaces: ``hb::band_ring::band_ring<hb::Bf16Io, 2>``
    -> ``band_ring_bf16<2>``; ``hb::dense_attend_f32<64>`` stays as it is); other kernels keep a short prefix."""
    m = re.search(r"hb::(?:\w+::)*(\w+)(?:<([^()<>]*)>)?", name)
    if m:
        base, args = m.group(1), [a.strip() for a in (m.group(2) or "").split(",") if a.strip()]
        if args and args[0] in IO_SUFFIX:
            base, args = base + IO_SUFFIX[args[0]], args[1:]
        return base + (f"<{','.join(args)}>" if args else "")
    if "at::native::" in name:  # torch: the kernel template and the operation it applies
        head = re.search(r"at::native::(?:\(anonymous namespace\)::)?(\w+)", name)
        ops = re.findall(r"(\w+(?:Functor\w*|_kernel_cuda|Ops|_copy_kernel_cuda))", name[head.end():] if head else name)
        kinds = re.findall(r"c10::(BFloat16|Half)|<(float|double)", name)
        elem = next((a or b for a, b in kinds), "")
        label = head.group(1) if head else "torch"
        return f"torch {label}<{ops[0] if ops else ''}{', ' + elem if elem else ''}>"
    return name.split("(")[0][:60]


def kernel_stats(trace_dir: Path) -> dict[str, dict]:
    """Per short name: calls, average / min / max duration and share of GPU time, summed over the kernels that
    share the short name."""
    rows: dict[str, dict] = {}
    for r in csv.DictReader(open(trace_dir / "run_kernel_stats.csv")):
        k, calls = short_name(r["Name"]), int(r["Calls"])
        total = float(r["TotalDurationNs"]) / 1e3 if r.get("TotalDurationNs") else calls * float(r["AverageNs"]) / 1e3
        e = rows.setdefault(k, {"calls": 0, "total_us": 0.0, "min_us": float("inf"), "max_us": 0.0, "pct": 0.0})
        e["calls"] += calls
        e["total_us"] += total
        e["min_us"] = min(e["min_us"], float(r["MinNs"]) / 1e3)
        e["max_us"] = max(e["max_us"], float(r["MaxNs"]) / 1e3)
        e["pct"] += float(r["Percentage"])
    for e in rows.values():
        e["avg_us"] = e["total_us"] / max(e["calls"], 1)
    return rows


def counter(pmc_dir: Path, name: str) -> tuple[dict[str, float], float]:
    """Average counter value per dispatch for each kernel, and the value of the largest copy dispatch."""
    vals: dict[str, list[float]] = collections.defaultdict(list)
    copy = 0.0
    for r in csv.DictReader(open(pmc_dir / "run_counter_collection.csv")):
        if r["Counter_Name"] != name:
            continue
        v = float(r["Counter_Value"])
        k = short_name(r["Kernel_Name"])
        vals[k].append(v)
        if k == COPY_KERNEL:
            copy = max(copy, v)
    return {k: sum(v) / len(v) for k, v in vals.items()}, copy


def all_counters(pmc_dir: Path) -> dict[str, dict[str, float]]:
    """Average value per dispatch of every counter in a `--pmc` run, per kernel on the path."""
    vals: dict[tuple[str, str], list[float]] = collections.defaultdict(list)
    for r in csv.DictReader(open(pmc_dir / "run_counter_collection.csv")):
        k = short_name(r["Kernel_Name"])
        if k.startswith(("dense", "band")):
            vals[(k, r["Counter_Name"])].append(float(r["Counter_Value"]))
    out: dict[str, dict[str, float]] = collections.defaultdict(dict)
    for (k, c), v in vals.items():
        out[k][c] = sum(v) / len(v)
    return out


def agent(pmc_dir: Path) -> dict[str, int]:
    for r in csv.DictReader(open(pmc_dir / "run_agent_info.csv")):
        if r.get("Agent_Type") == "GPU":
            return {k: int(r[k]) for k in ("Simd_Count", "Num_Xcc", "Cu_Count")}
    raise SystemExit("no GPU agent in run_agent_info.csv")


def counter_section(dirs: list[Path]) -> list[str]:
    """Markdown table of the hardware counters of one or more `--pmc` passes, with the derived fractions whose inputs
    were collected: matrix-core busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE / XCDs) (GRBM_GUI_ACTIVE is
    summed over the XCDs, the busy cycles over the SIMDs); LDS bank-conflict cycles per LDS-active cycle; and, per
    wave-cycle (SQ_WAVE_CYCLES), the cycles a wave has a VALU instruction in flight (SQ_ACTIVE_INST_VALU), waits on a
    dependency or counter (SQ_WAIT_ANY) and waits for its next instruction to issue (SQ_WAIT_INST_ANY); and the share
    of matrix-core busy cycles with VALU work executing beside them (SQ_VALU_MFMA_COEXEC_CYCLES)."""
    merged: dict[str, dict[str, float]] = collections.defaultdict(dict)
    info = agent(dirs[0])
    for d in dirs:
        for k, cs in all_counters(d).items():
            merged[k].update(cs)
    names = sorted({c for cs in merged.values() for c in cs})

    def busy(cs):
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in cs or not cs.get("GRBM_GUI_ACTIVE"):
            return None
        return cs["SQ_VALU_MFMA_BUSY_CYCLES"] / (info["Simd_Count"] * cs["GRBM_GUI_ACTIVE"] / info["Num_Xcc"])

    def ratio(num, den):
        return lambda cs: cs[num] / cs[den] if num in cs and cs.get(den) else None
    derived = [("MFMA busy", busy), ("LDS bank conflict / LDS active", ratio("SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE")),
               ("VALU active / wave cycles", ratio("SQ_ACTIVE_INST_VALU", "SQ_WAVE_CYCLES")),
               ("waiting / wave cycles", ratio("SQ_WAIT_ANY", "SQ_WAVE_CYCLES")),
               ("waiting to issue / wave cycles", ratio("SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES")),
               ("VALU beside MFMA / MFMA busy", ratio("SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES"))]
    derived = [(n, f) for n, f in derived if any(f(cs) is not None for cs in merged.values())]
    lines = ["", "## Hardware counters (`--pmc`; average per dispatch, summed over the GPU)", "",
             f"GPU: {info['Cu_Count']} CUs, {info['Simd_Count']} SIMDs, {info['Num_Xcc']} XCDs.", "",
             "| kernel | " + " | ".join(names + [n for n, _ in derived]) + " |",
             "|---|" + "---|" * (len(names) + len(derived))]
    for k in sorted(merged):
        cs = merged[k]
        vals = [f"{cs[c]:.4g}" if c in cs else "-" for c in names]
        vals += [f"{v:.1%}" if (v := f(cs)) is not None else "-" for _, f in derived]
        lines.append(f"| `{k}` | " + " | ".join(vals) + " |")
    return lines


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--trace", type=Path, required=True)
    ap.add_argument("--fetch", type=Path)
    ap.add_argument("--write", type=Path)
    ap.add_argument("--pmc", type=Path, action="append", default=[],
                    help="a --pmc run with other counters (repeatable); tabulated with derived fractions")
    ap.add_argument("--copy-bytes", type=int, default=1 << 28)
    ap.add_argument("--algorithmic", action="append", default=[], metavar="KERNEL=BYTES",
                    help="algorithmic bytes per launch, for the traffic/algorithmic ratio")
    ap.add_argument("--command", action="append", default=[], help="command lines to quote in the summary")
    ap.add_argument("--title", default="rocprofv3 summary")
    ap.add_argument("--md", type=Path, required=True)
    ap.add_argument("--json", type=Path)
    args = ap.parse_args()

    stats = kernel_stats(args.trace)
    algo = {k: float(v) for k, v in (a.split("=", 1) for a in args.algorithmic)}
    lines = [f"# {args.title}", "", "Commands (from the repository root on the GPU host):", "", "```"]
    lines += args.command + ["```", "", "## Kernel trace (`--kernel-trace --stats`)", "",
                             "| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|"]
    for k, s in sorted(stats.items(), key=lambda kv: -kv[1]["pct"]):
        lines.append(f"| `{k}` | {s['calls']} | {s['avg_us']:.2f} | {s['min_us']:.2f} | {s['max_us']:.2f} "
                     f"| {s['pct']:.2f} |")

    traffic = {}
    if args.fetch and args.write:
        fetch, copy_fetch = counter(args.fetch, "FETCH_SIZE")
        write, copy_write = counter(args.write, "WRITE_SIZE")
        if copy_fetch <= 0 or copy_write <= 0:
            raise SystemExit(f"no {COPY_KERNEL} dispatch found for calibration")
        ff = args.copy_bytes / 1024 / copy_fetch
        wf = args.copy_bytes / 1024 / copy_write
        lines += ["", "## HBM traffic (`--pmc FETCH_SIZE`, `--pmc WRITE_SIZE`; KiB per dispatch)", "",
                  f"Calibration: a {args.copy_bytes >> 20} MiB device copy reads FETCH_SIZE = {copy_fetch:.0f} KiB "
                  f"and WRITE_SIZE = {copy_write:.0f} KiB, so bytes = FETCH_SIZE x {ff:.3f} x 1024 and "
                  f"WRITE_SIZE x {wf:.3f} x 1024.", "",
                  "| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes / launch | algorithmic bytes | ratio |",
                  "|---|---|---|---|---|---|"]
        for k in sorted(set(fetch) & set(write)):
            if not k.startswith(("dense", "band", "rope")):
                continue
            total = (fetch[k] * ff + write[k] * wf) * 1024
            traffic[k] = total
            a = algo.get(k)
            tail = f"{a:.4g} | {total / a:.2f} |" if a else "- | - |"
            lines.append(f"| `{k}` | {fetch[k]:.0f} | {write[k]:.0f} | {total:.4g} | {tail}")
    if args.pmc:
        lines += counter_section(args.pmc)
    args.md.write_text("\n".join(lines) + "\n")
    if args.json is not None:
        args.json.write_text(json.dumps({"hbm_bytes_per_launch": {k: round(v) for k, v in traffic.items()},
                                         "avg_us": {k: round(s["avg_us"], 2) for k, s in stats.items()
                                                    if k.startswith(("dense", "band", "rope"))},
                                         "commands": args.command}, indent=1) + "\n")
    print(args.md.read_text())
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
