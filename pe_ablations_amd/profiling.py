"""rocprofv3 post-processing for the PE-attention kernels (MI355X).

Subcommands (run from the repository root):

  python -m pe_ablations_amd.profiling copy
      Calibration workload: a plain 1 GiB fp32 device copy, three times.  Profiled under
      ``rocprofv3 --pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE`` it gives the factor between each
      counter and the bytes a kernel really moves (the copy reads and writes exactly 1 GiB).

  python -m pe_ablations_amd.profiling stats DIR OUT.md --title T --cmd C [--note N]
      Markdown table of a ``rocprofv3 --kernel-trace --stats -o run -f csv -d DIR`` run.

  python -m pe_ablations_amd.profiling traffic --copy-fetch D --copy-write D --fetch D --write D \\
          --out OUT.json [--md OUT.md --cmd C ...]
      HBM bytes per dispatch of every library kernel: the median FETCH_SIZE / WRITE_SIZE (KiB per
      dispatch) of the workload runs, each scaled by the calibration copy's factor.

  python -m pe_ablations_amd.profiling counters OUT.md DIR [DIR ...] --title T [--cmd C ...]
      Median per-dispatch value of every counter of ``rocprofv3 --pmc`` runs, per library kernel.
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import statistics
import sys

GIB = 1 << 30


def _kernel_key(name: str) -> str:
    """'void pe::dkdv_bf16_kernel<256, 128, 4>(pe::CoreArgs)' -> 'dkdv_bf16_kernel<256, 128, 4>'."""
    n = name.strip()
    if n.startswith("void "):
        n = n[5:]
    depth = 0
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            n = n[:i]
            break
    return n.replace("pe::", "")


def _counter_rows(d: str):
    path = os.path.join(d, "run_counter_collection.csv")
    with open(path) as f:
        return list(csv.DictReader(f))


def _per_kernel(d: str, counter: str, library_only: bool = False) -> dict:
    """{kernel: [counter value per dispatch]} (values of one dispatch summed over its rows)."""
    acc: dict = {}
    for r in _counter_rows(d):
        if r["Counter_Name"] != counter or (library_only and "pe::" not in r["Kernel_Name"]):
            continue
        per = acc.setdefault(_kernel_key(r["Kernel_Name"]), {})
        did = r.get("Dispatch_Id", "0")
        per[did] = per.get(did, 0.0) + float(r["Counter_Value"])
    return {k: list(v.values()) for k, v in acc.items()}


def _copy_factor(d: str, counter: str) -> tuple[float, float]:
    """(bytes per counted KiB, median counter KiB) of the calibration copy's dispatches."""
    vals = [v for k, vs in _per_kernel(d, counter).items() if "copy" in k.lower() or "elementwise" in k.lower()
            for v in vs if v > 0]
    if not vals:
        raise SystemExit(f"no copy dispatch with {counter} in {d}")
    big = [v for v in vals if v > 0.25 * max(vals)]  # the 1 GiB copies, not allocator fills
    med = statistics.median(big)
    return GIB / (med * 1024.0), med


def cmd_copy(_args) -> int:
    import torch
    n = GIB // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(f"copied {n * 4} bytes x3", flush=True)
    return 0


def cmd_stats(args) -> int:
    with open(os.path.join(args.dir, "run_kernel_stats.csv")) as f:
        rows = list(csv.DictReader(f))
    lines = [f"# {args.title}", "", "Command (repository root on one MI355X):", "", "```", args.cmd, "```", ""]
    if args.note:
        lines += [args.note, ""]
    # per-kernel average over the dispatches after the first `skip` (the warm-up calls), in order
    durs: dict = {}
    trace = os.path.join(args.dir, "run_kernel_trace.csv")
    if args.skip and os.path.exists(trace):
        with open(trace) as f:
            for r in sorted(csv.DictReader(f), key=lambda r: int(r["Dispatch_Id"])):
                durs.setdefault(r["Kernel_Name"], []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    head = "| kernel | calls | avg us | min us | max us | total ms | % |"
    if durs:
        head += f" avg us after {args.skip} calls |"
    lines += [head, "|" + "---|" * (head.count("|") - 1)]
    for r in rows:
        line = (f"| {_kernel_key(r['Name'])[:70]} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.2f} |")
        if durs:
            d = durs.get(r["Name"], [])[args.skip:]
            line += f" {sum(d) / len(d) / 1e3:.1f} |" if d else " |"
        lines.append(line)
    with open(args.out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {args.out}")
    return 0


def cmd_traffic(args) -> int:
    ff, fmed = _copy_factor(args.copy_fetch, "FETCH_SIZE")
    wf, wmed = _copy_factor(args.copy_write, "WRITE_SIZE")
    fetch = _per_kernel(args.fetch, "FETCH_SIZE", library_only=True)
    write = _per_kernel(args.write, "WRITE_SIZE", library_only=True)
    kernels = {}
    for k in sorted(set(fetch) | set(write)):
        fv, wv = fetch.get(k, []), write.get(k, [])
        kernels[k] = {
            "dispatches": max(len(fv), len(wv)),
            "fetch_kib_counted": statistics.median(fv) if fv else None,
            "write_kib_counted": statistics.median(wv) if wv else None,
            "fetch_bytes": statistics.median(fv) * 1024.0 * ff if fv else None,
            "write_bytes": statistics.median(wv) * 1024.0 * wf if wv else None,
        }
    out = {
        "calibration": {"copy_bytes": GIB, "fetch_kib_counted": fmed, "write_kib_counted": wmed,
                        "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
        "kernels": kernels,
        "commands": args.cmd or [],
    }
    with open(args.out, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {args.out}")
    if args.md:
        lines = [f"# {args.title}", "", "Commands (repository root on one MI355X):", "", "```"] + (args.cmd or []) + [
            "```", "",
            f"Calibration: a 1 GiB fp32 copy reads FETCH_SIZE = {fmed:.0f} KiB and WRITE_SIZE = {wmed:.0f} KiB per "
            f"dispatch, so bytes = FETCH_SIZE x 1024 x {ff:.3f} and WRITE_SIZE x 1024 x {wf:.3f}.", "",
            "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM read GB | HBM write GB |",
            "|---|---|---|---|---|---|"]
        def num(x, fmt):
            return "" if x is None else format(x, fmt)

        for k, v in kernels.items():
            gb_r = None if v["fetch_bytes"] is None else v["fetch_bytes"] / 1e9
            gb_w = None if v["write_bytes"] is None else v["write_bytes"] / 1e9
            lines.append(f"| {k[:70]} | {v['dispatches']} | {num(v['fetch_kib_counted'], '.0f')} | "
                         f"{num(v['write_kib_counted'], '.0f')} | {num(gb_r, '.3f')} | {num(gb_w, '.3f')} |")
        with open(args.md, "w") as f:
            f.write("\n".join(lines) + "\n")
        print(f"wrote {args.md}")
    return 0


def cmd_counters(args) -> int:
    """Markdown table: median per-dispatch value of every counter found in the given runs."""
    table: dict = {}
    names: list = []
    for d in args.dirs:
        for r in _counter_rows(d):
            if r["Counter_Name"] not in names:
                names.append(r["Counter_Name"])
        for c in list(names):
            for k, vals in _per_kernel(d, c, library_only=True).items():
                table.setdefault(k, {})[c] = statistics.median(vals)
    lines = [f"# {args.title}", "", "Commands (repository root on one MI355X):", "", "```"] + (args.cmd or []) + [
        "```", ""]
    if args.note:
        lines += [args.note, ""]
    lines += ["| kernel | " + " | ".join(names) + " |", "|---|" + "---|" * len(names)]
    for k, v in sorted(table.items()):
        lines.append(f"| {k[:50]} | " + " | ".join(format(v[c], ".4g") if c in v else "" for c in names) + " |")
    with open(args.out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {args.out}")
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd_name", required=True)
    sub.add_parser("copy")
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("out")
    s.add_argument("--title", required=True)
    s.add_argument("--cmd", required=True)
    s.add_argument("--note", default="")
    s.add_argument("--skip", type=int, default=0, help="also average each kernel after its first N calls")
    t = sub.add_parser("traffic")
    for n in ("copy-fetch", "copy-write", "fetch", "write", "out"):
        t.add_argument("--" + n, required=True)
    t.add_argument("--md", default="")
    t.add_argument("--title", default="HBM traffic per dispatch")
    t.add_argument("--cmd", action="append")
    c = sub.add_parser("counters")
    c.add_argument("out")
    c.add_argument("dirs", nargs="+")
    c.add_argument("--title", required=True)
    c.add_argument("--cmd", action="append")
    c.add_argument("--note", default="")
    args = ap.parse_args(argv)
    if args.cmd_name == "counters":
        return cmd_counters(args)
    if args.cmd_name == "copy":
        return cmd_copy(args)
    if args.cmd_name == "stats":
        return cmd_stats(args)
    return cmd_traffic(args)


if __name__ == "__main__":
    sys.exit(main())
