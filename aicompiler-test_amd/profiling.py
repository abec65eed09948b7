"""Summaries of rocprofv3 results for the gfx950 decode backend.

Two subcommands over the rocpd SQLite databases rocprofv3 writes:

  summary  kernel-trace table (per kernel and grid: calls, average / median /
           min / max duration, VGPR, AGPR, LDS) as markdown;
  traffic  HBM bytes per launch of one kernel from two counter runs
           (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by
           what the same counter reads for the plain copy probe of known size
           (tmc_copy_bytes) in the same run, written as JSON.

Example (MI355X, repo root):
  rocprofv3 --pmc FETCH_SIZE -d out/f -o run -- python3 bench.py --no-extra --no-cpu
  rocprofv3 --pmc WRITE_SIZE -d out/w -o run -- python3 bench.py --no-extra --no-cpu
  python3 aicompiler-test_amd/profiling.py traffic --fetch out/f/run_results.db \\
      --write out/w/run_results.db --kernel gemv_dot_kernel --template Li2ELi1ELi1ELi2ELi4E \\
      --copy-bytes 268435456 --algorithmic 180385280 --out profiles/gate_up_traffic.json
"""
from __future__ import annotations

import argparse
import collections
import json
import re
import sqlite3
import statistics
import sys


def short_name(name: str) -> str:
    m = re.search(r"tmc::\(anonymous namespace\)::(\w+)(<[^>]*>)?", name)
    if m:
        return m.group(1) + (m.group(2) or "")
    m = re.search(r"GLOBAL__N_1\d+(\w+?)I(.*)EEv", name)
    if m:
        return m.group(1) + " [" + m.group(2)[:40] + "]"
    return name[:60]


def kernel_summary(db: str, title: str, command: str) -> str:
    con = sqlite3.connect(db)
    rows = con.execute("select name, grid_x, grid_y, grid_z, workgroup_x, vgpr_count, "
                       "accum_vgpr_count, lds_size, duration from kernels").fetchall()
    agg, meta = collections.defaultdict(list), {}
    for name, gx, gy, gz, wx, vgpr, agpr, lds, dur in rows:
        key = (name, f"{gx}x{gy}x{gz}", wx)
        agg[key].append(dur / 1000.0)
        meta[key] = (vgpr, agpr, lds)
    out = [f"# {title}", "", "Command (repo root, MI355X box):", "", f"    {command}", "",
           "Durations in microseconds from the kernel trace (`kernels` view of the rocpd "
           "database).", "",
           "| kernel | grid (threads) | block | VGPR | AGPR | LDS B | calls | avg | median | min | max |",
           "|---|---|---|---|---|---|---|---|---|---|---|"]
    for key, d in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        if len(d) < 2:
            continue
        vgpr, agpr, lds = meta[key]
        out.append(f"| `{short_name(key[0])}` | {key[1]} | {key[2]} | {vgpr} | {agpr} | {lds} | "
                   f"{len(d)} | {statistics.mean(d):.2f} | {statistics.median(d):.2f} | "
                   f"{min(d):.2f} | {max(d):.2f} |")
    return "\n".join(out) + "\n"


def counter_per_dispatch(db: str, counter: str) -> dict:
    """kernel name -> list of per-dispatch values of `counter`."""
    con = sqlite3.connect(db)
    rows = con.execute("select kernel_name, counter_name, value from counters_collection"
                       ).fetchall()
    out = collections.defaultdict(list)
    for name, cname, value in rows:
        if cname == counter:
            out[name].append(float(value))
    return out


def _mean_for(values: dict, kernel: str, template: str | None) -> tuple:
    picked = [v for name, vs in values.items() if kernel in name and
              (template is None or template in name) for v in vs]
    if not picked:
        raise SystemExit(f"no dispatch of {kernel} {template or ''} in the database")
    return statistics.mean(picked), len(picked)


def traffic(fetch_db: str, write_db: str, kernel: str, template: str | None, copy_bytes: int,
            algorithmic: int | None) -> dict:
    fetch = counter_per_dispatch(fetch_db, "FETCH_SIZE")
    write = counter_per_dispatch(write_db, "WRITE_SIZE")
    copy_fetch, n_cf = _mean_for(fetch, "copy_kernel", None)
    copy_write, n_cw = _mean_for(write, "copy_kernel", None)
    k_fetch, n_kf = _mean_for(fetch, kernel, template)
    k_write, n_kw = _mean_for(write, kernel, template)
    f_scale = copy_bytes / (copy_fetch * 1024.0)   # bytes per counted KiB
    w_scale = copy_bytes / (copy_write * 1024.0)
    read_bytes = k_fetch * 1024.0 * f_scale
    written_bytes = k_write * 1024.0 * w_scale
    result = {
        "kernel": kernel + (f" [{template}]" if template else ""),
        "fetch_kib_per_dispatch": round(k_fetch, 1), "write_kib_per_dispatch": round(k_write, 1),
        "dispatches": {"kernel_fetch": n_kf, "kernel_write": n_kw, "copy_fetch": n_cf,
                       "copy_write": n_cw},
        "copy_probe_bytes": copy_bytes,
        "copy_fetch_kib": round(copy_fetch, 1), "copy_write_kib": round(copy_write, 1),
        "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
        "read_bytes_per_launch": int(read_bytes), "written_bytes_per_launch": int(written_bytes),
        "traffic_bytes_per_launch": int(read_bytes + written_bytes),
    }
    if algorithmic:
        result["algorithmic_bytes_per_launch"] = algorithmic
        result["traffic_over_algorithmic"] = round((read_bytes + written_bytes) / algorithmic, 4)
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("summary")
    s.add_argument("db")
    s.add_argument("--title", required=True)
    s.add_argument("--command", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--template")
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--algorithmic", type=int)
    t.add_argument("--command", default="")
    t.add_argument("--out")
    a = ap.parse_args(argv)
    if a.cmd == "summary":
        sys.stdout.write(kernel_summary(a.db, a.title, a.command))
        return 0
    result = traffic(a.fetch, a.write, a.kernel, a.template, a.copy_bytes, a.algorithmic)
    if a.command:
        result["command"] = a.command
    text = json.dumps(result, indent=2) + "\n"
    if a.out:
        with open(a.out, "w") as f:
            f.write(text)
    sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
