"""Summaries of rocprofv3 output for profiles/ (run on the CPU host after a GPU run).

Three subcommands, each reading rocprofv3's CSV output (``--output-format csv
-o run``) and writing a short Markdown summary:

  trace DIR              kernel statistics of a ``--kernel-trace --stats`` run
                         (DIR/run_kernel_stats.csv)
  traffic FETCH WRITE    HBM bytes per launch of one kernel from two ``--pmc``
                         runs (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch),
                         each scaled by what the same counter reads for the
                         plain copy kernel of 1 GiB that ``bench.py --pmc-run``
                         launches (molot_probe_copy); also records the result
                         in profiles/traffic.json under the config's name,
                         stamped with the hash of the kernel source it was
                         measured on, so bench.py can tell a stale entry
  counters DIR...        per-dispatch means of any counters, per kernel

Every summary starts with the commands that made it (given with --cmd).
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import os
import re
import sys
from collections import defaultdict

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNEL_SOURCE = os.path.join(ROOT, "molot_amd", "csrc", "attn_decode.hip")
COPY_BYTES = 1 << 30  # bench.py --pmc-run: molot_probe_copy of 1 GiB


def source_hash() -> str:
    """sha256 (first 16 hex digits) of the kernel source a measurement belongs to."""
    with open(KERNEL_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def short_name(name: str, width: int = 110) -> str:
    n = name.replace("(anonymous namespace)::", "")
    n = re.sub(r"\(AttnArgs\)$|\(PfArgs\)$|\(CombArgs\)$", "", n)
    return n if len(n) <= width else n[:width - 3] + "..."


def _rows(path: str):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _find(d: str, suffix: str) -> str:
    for fn in sorted(os.listdir(d)):
        if fn.endswith(suffix):
            return os.path.join(d, fn)
    raise FileNotFoundError(f"no *{suffix} in {d}")


def _cmd_block(cmds) -> str:
    return "```\n" + "\n".join(cmds) + "\n```\n" if cmds else ""


def _source_line() -> str:
    return (f"Kernel source: `molot_amd/csrc/attn_decode.hip`, sha256[:16] `{source_hash()}` "
            "(the tree the summary was written from).\n")


def trace(args) -> str:
    rows = _rows(_find(args.dir, "_kernel_stats.csv"))
    out = [f"# {args.title}\n", "Commands (repository root of the GPU box):\n",
           _cmd_block(args.cmd), _source_line(), args.note + "\n" if args.note else "",
           "| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in rows[: args.top]:
        out.append(f"| `{short_name(r['Name'])}` | {r['Calls']} | "
                   f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                   f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")
    if args.log:
        lines = [ln.rstrip() for ln in open(args.log) if ln.startswith("[bench]")]
        js = [ln.rstrip() for ln in open(args.log) if ln.startswith("{")]
        out += ["", args.log_title, "", "```"]
        out += lines + js[-1:] + ["```"]
    return "\n".join(out) + "\n"


def _per_dispatch(d: str, counter: str):
    """counter -> kernel name -> list of per-dispatch values."""
    vals = defaultdict(list)
    for r in _rows(_find(d, "_counter_collection.csv")):
        if r["Counter_Name"] == counter:
            vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return vals


def _pick(vals, pattern: str):
    keys = [k for k in vals if re.search(pattern, k)]
    if not keys:
        raise KeyError(f"no kernel matching {pattern!r} among {sorted(vals)}")
    xs = [x for k in keys for x in vals[k]]
    return sum(xs) / len(xs), len(xs), keys


def traffic(args) -> str:
    fetch = _per_dispatch(args.fetch, "FETCH_SIZE")
    write = _per_dispatch(args.write, "WRITE_SIZE")
    f_k, f_n, names = _pick(fetch, args.kernel)
    w_k, w_n, _ = _pick(write, args.kernel)
    f_c, fc_n, _ = _pick(fetch, r"copy_kernel")
    w_c, wc_n, _ = _pick(write, r"copy_kernel")
    f_cal = COPY_BYTES / 1024 / f_c  # bytes per counted KiB, as the copy's read says
    w_cal = COPY_BYTES / 1024 / w_c
    fb = f_k * 1024 * f_cal
    wb = w_k * 1024 * w_cal
    total = fb + wb
    entry = {
        "kernel": short_name(names[0], 200),
        "fetch_kib_per_launch_raw": round(f_k, 1),
        "write_kib_per_launch_raw": round(w_k, 1),
        "fetch_calibration": round(f_cal, 4),
        "write_calibration": round(w_cal, 4),
        "fetch_bytes_per_launch": int(round(fb)),
        "write_bytes_per_launch": int(round(wb)),
        "traffic_bytes_per_launch": int(round(total)),
        "algorithmic_bytes_per_launch": args.algorithmic,
        "source_sha256": source_hash(),
    }
    if args.second:
        s_f, _, _ = _pick(fetch, args.second)
        s_w, _, _ = _pick(write, args.second)
        entry["second_kernel"] = args.second
        entry["second_kernel_traffic_bytes_per_launch"] = int(round(
            s_f * 1024 * f_cal + s_w * 1024 * w_cal))
    if args.json:
        data = {}
        if os.path.exists(args.json):
            with open(args.json) as f:
                data = json.load(f)
        data[args.config] = entry
        with open(args.json, "w") as f:
            json.dump(data, f, indent=1, sort_keys=True)
            f.write("\n")
    ratio = total / args.algorithmic if args.algorithmic else float("nan")
    out = [f"# {args.title}\n", "Commands (repository root of the GPU box):\n", _cmd_block(args.cmd),
           _source_line(),
           "`bench.py --pmc-run` launches eager steps, then three copies of 1 GiB through "
           "`molot_probe_copy` (a plain copy kernel), whose readings calibrate the counters.\n",
           "| counter | kernel KiB/dispatch (n) | copy_kernel KiB/dispatch (n) | bytes per counted KiB |",
           "|---|---|---|---|",
           f"| FETCH_SIZE | {f_k:.1f} ({f_n}) | {f_c:.1f} ({fc_n}) | {f_cal * 1024:.1f} |",
           f"| WRITE_SIZE | {w_k:.1f} ({w_n}) | {w_c:.1f} ({wc_n}) | {w_cal * 1024:.1f} |", "",
           f"Kernel: `{short_name(names[0])}`", "",
           f"Calibrated traffic per launch: fetch {fb / 1e6:.3f} MB + write {wb / 1e6:.3f} MB = "
           f"**{total / 1e6:.3f} MB**, against {args.algorithmic / 1e6:.3f} MB algorithmic "
           f"(ratio {ratio:.4f}).", ""]
    if args.note:
        out.append(args.note)
    return "\n".join(out) + "\n"


def counters(args) -> str:
    table = defaultdict(dict)  # kernel -> counter -> (mean, n)
    names = set()
    for d in args.dirs:
        rows = _rows(_find(d, "_counter_collection.csv"))
        for ctr in sorted({r["Counter_Name"] for r in rows}):
            vals = _per_dispatch(d, ctr)
            for k, xs in vals.items():
                if re.search(args.kernel, k):
                    table[k][ctr] = (sum(xs) / len(xs), len(xs))
                    names.add(ctr)
    cols = sorted(names)
    out = [f"# {args.title}\n", "Commands (repository root of the GPU box):\n", _cmd_block(args.cmd),
           _source_line(), "Per-dispatch means (number of dispatches in parentheses).\n",
           "| kernel | " + " | ".join(cols) + " |", "|---|" + "---|" * len(cols)]
    for k in sorted(table):
        cells = [f"{table[k][c][0]:.4g} ({table[k][c][1]})" if c in table[k] else "" for c in cols]
        out.append(f"| `{short_name(k)}` | " + " | ".join(cells) + " |")
    for ratio in args.ratio or []:
        a, b = ratio.split("/")
        for k in sorted(table):
            if a in table[k] and b in table[k] and table[k][b][0]:
                out.append(f"\n`{short_name(k, 60)}`: {a} / {b} = "
                           f"{table[k][a][0] / table[k][b][0]:.3f}")
    if args.note:
        out += ["", args.note]
    return "\n".join(out) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="what", required=True)
    common = argparse.ArgumentParser(add_help=False)
    common.add_argument("--title", required=True)
    common.add_argument("--cmd", action="append", default=[], help="a command that made the data")
    common.add_argument("--note", default="")
    common.add_argument("--out", required=True, help="Markdown summary to write")
    t = sub.add_parser("trace", parents=[common])
    t.add_argument("dir")
    t.add_argument("--top", type=int, default=8)
    t.add_argument("--log", help="bench.py output (stderr lines + JSON line) to append")
    t.add_argument("--log-title", default="The same command without the profiler (bench.py's "
                   "stderr lines and JSON line):")
    r = sub.add_parser("traffic", parents=[common])
    r.add_argument("fetch")
    r.add_argument("write")
    r.add_argument("--kernel", required=True, help="regex of the kernel's name")
    r.add_argument("--second", help="regex of a second kernel of the step (the combine)")
    r.add_argument("--config", required=True)
    r.add_argument("--algorithmic", type=int, required=True)
    r.add_argument("--json", default=os.path.join(ROOT, "profiles", "traffic.json"))
    c = sub.add_parser("counters", parents=[common])
    c.add_argument("dirs", nargs="+")
    c.add_argument("--kernel", default=".", help="regex of the kernels to list")
    c.add_argument("--ratio", action="append", help="A/B ratios of counters to print")
    a = ap.parse_args(argv)
    text = {"trace": trace, "traffic": traffic, "counters": counters}[a.what](a)
    with open(a.out, "w") as f:
        f.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
