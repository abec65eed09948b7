"""Summaries of rocprofv3 results for the gfx950 decode backend.

Subcommands over the rocpd SQLite databases rocprofv3 writes:

  summary  kernel-trace table (per kernel and grid: calls, average / median /
           min / max duration, VGPR, AGPR, LDS) as markdown;
  traffic  HBM bytes per launch of one kernel from two counter runs
           (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by
           what the same counter reads for the plain copy probe of known size
           (tmc_copy_bytes) in the same run, written as JSON;
  table    every kernel of a run (calls and average duration from a kernel
           trace; HBM bytes per dispatch from the FETCH_SIZE, WRITE_SIZE and
           EA read-request passes, the first two scaled by the copy probe);
           optional algorithmic bytes per kernel; markdown and JSON;
  mfma     MfmaUtil and the f16 MFMA operation count per dispatch of every
           kernel that issues MFMA, with achieved TFLOP/s from the trace;
  stalls   issue and stall counters (SQ wave / wait / issue cycles, VMEM
           latency, occupancy, TA busy, TCP-to-L2 request latency, address
           translation) per dispatch of chosen kernels, with per-wave ratios;
  c4       the C4 record: the paged attention kernel and the gather probe
           over the same bytes, their traffic rows (from `table --json`) and
           stall rows (from `stalls --json`) side by side.

FETCH_SIZE on gfx950 counts each 128-byte EA read request as 64 bytes (its
expression adds TCC_BUBBLE x 128, and TCC_BUBBLE stays 0), so a read-heavy
kernel's FETCH_SIZE is half its bytes; the copy probe calibrates the factor,
and the EA request counters (TCC_EA0_RDREQ_32B/64B/128B: 32, 64 and 128
bytes per request) give the read bytes without a scale, as a cross-check.

Example (MI355X, repo root):
  rocprofv3 --pmc FETCH_SIZE -d out/f -o run -- python3 bench.py --no-extra --no-cpu
  rocprofv3 --pmc WRITE_SIZE -d out/w -o run -- python3 bench.py --no-extra --no-cpu
  python3 aicompiler-test_amd/profiling.py traffic --fetch out/f/run_results.db \\
      --write out/w/run_results.db --kernel gemv_norm_kernel --template Li2ELi1ELi2EDF16_Li1E \\
      --copy-bytes 268435456 --algorithmic 180409856 --out profiles/norm_gate_up_traffic.json
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
    m = re.search(r"(?:tmc::)?\(anonymous namespace\)::(\w+)(<[^>]*>)?", name)
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


def _per_kernel(db: str, counters: tuple) -> dict:
    """(short name, grid) -> {counter: [per-dispatch values]} from a
    counters_collection database."""
    con = sqlite3.connect(db)
    rows = con.execute("select kernel_name, grid_size_x, grid_size_y, grid_size_z, counter_name, "
                       "value from counters_collection").fetchall()
    out = collections.defaultdict(lambda: collections.defaultdict(list))
    for name, gx, gy, gz, cname, value in rows:
        if cname in counters:
            out[(short_name(name), f"{gx}x{gy}x{gz}")][cname].append(float(value))
    return out


def _trace(db: str) -> dict:
    """(short name, grid) -> list of durations in microseconds."""
    con = sqlite3.connect(db)
    out = collections.defaultdict(list)
    for name, gx, gy, gz, dur in con.execute(
            "select name, grid_x, grid_y, grid_z, duration from kernels").fetchall():
        out[(short_name(name), f"{gx}x{gy}x{gz}")].append(dur / 1000.0)
    return out


def _mean(values: list) -> float:
    return statistics.mean(values) if values else float("nan")


def _copy_scale(per_kernel: dict, counter: str, copy_bytes: int) -> float:
    vals = [v for (name, _), d in per_kernel.items() if name.startswith("copy_kernel")
            for v in d.get(counter, [])]
    if not vals:
        raise SystemExit(f"no copy_kernel dispatch with {counter} in the database")
    return copy_bytes / (statistics.mean(vals) * 1024.0)


def _algorithmic(specs: list) -> list:
    """'name_substring[@grid]=bytes' -> [(substring, grid or None, bytes)]."""
    out = []
    for spec in specs or []:
        key, value = spec.rsplit("=", 1)
        name, _, grid = key.partition("@")
        out.append((name, grid or None, int(float(value))))
    return out


def traffic_table(fetch_db: str, write_db: str, rdreq_db: str, trace_db: str, copy_bytes: int,
                  min_calls: int, algorithmic: list, hit_db: str | None = None) -> list:
    fetch = _per_kernel(fetch_db, ("FETCH_SIZE",))
    write = _per_kernel(write_db, ("WRITE_SIZE",))
    rd = _per_kernel(rdreq_db, ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum",
                                "TCC_EA0_RDREQ_128B_sum"))
    trace = _trace(trace_db)
    hits = _per_kernel(hit_db, ("TCC_HIT_sum", "TCC_MISS_sum")) if hit_db else {}
    f_scale = _copy_scale(fetch, "FETCH_SIZE", copy_bytes)
    w_scale = _copy_scale(write, "WRITE_SIZE", copy_bytes)
    algo = _algorithmic(algorithmic)
    rows = []
    for key, durs in trace.items():
        if len(durs) < min_calls or key not in fetch or key not in write:
            continue
        name, grid = key
        f = _mean(fetch[key]["FETCH_SIZE"]) * 1024.0 * f_scale
        w = _mean(write[key]["WRITE_SIZE"]) * 1024.0 * w_scale
        r = rd.get(key, {})
        ea = None
        if r:
            ea = (32 * _mean(r.get("TCC_EA0_RDREQ_32B_sum", [0.0])) +
                  64 * _mean(r.get("TCC_EA0_RDREQ_64B_sum", [0.0])) +
                  128 * _mean(r.get("TCC_EA0_RDREQ_128B_sum", [0.0])))
        us = _mean(durs)
        row = {"kernel": name, "grid": grid, "calls": len(durs), "avg_us": round(us, 3),
               "read_bytes": int(f), "ea_read_bytes": None if ea is None else int(ea),
               "written_bytes": int(w),
               "achieved_gbps": round((f + w) / (us * 1e3), 1)}
        h = hits.get(key, {})
        if h:
            hit, miss = _mean(h.get("TCC_HIT_sum", [0.0])), _mean(h.get("TCC_MISS_sum", [0.0]))
            row["l2_hit_pct"] = round(100.0 * hit / (hit + miss), 2) if hit + miss else None
        for sub, g, b in algo:
            if sub in name and (g is None or g == grid):
                row["algorithmic_bytes"] = b
                row["traffic_over_algorithmic"] = round((f + w) / b, 4)
                row["algorithmic_gbps"] = round(b / (us * 1e3), 1)
        rows.append(row)
    rows.sort(key=lambda x: -x["avg_us"] * x["calls"])
    return [{"fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4)}] + rows


def table_markdown(rows: list, title: str, command: str) -> str:
    scales, rows = rows[0], rows[1:]
    out = [f"# {title}", "", "Commands (repo root, MI355X box):", "", f"    {command}", "",
           f"FETCH_SIZE scale {scales['fetch_scale']} and WRITE_SIZE scale "
           f"{scales['write_scale']} (bytes per counted byte, from the 256 MiB copy probe). "
           "`EA read` = 32/64/128 x the TCC_EA0_RDREQ_32B/64B/128B requests per dispatch "
           "(no scale). GB/s = (read + written) / average duration of the kernel trace.", "",
           "| kernel | grid | calls | avg us | read MB | EA read MB | written MB | GB/s | "
           "L2 hit % | algorithmic MB | traffic / algorithmic |",
           "|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        ea = "" if r["ea_read_bytes"] is None else f"{r['ea_read_bytes'] / 1e6:.3f}"
        alg = f"{r['algorithmic_bytes'] / 1e6:.3f}" if "algorithmic_bytes" in r else ""
        ratio = str(r.get("traffic_over_algorithmic", ""))
        out.append(f"| `{r['kernel']}` | {r['grid']} | {r['calls']} | {r['avg_us']:.2f} | "
                   f"{r['read_bytes'] / 1e6:.3f} | {ea} | {r['written_bytes'] / 1e6:.3f} | "
                   f"{r['achieved_gbps']} | {r.get('l2_hit_pct', '')} | {alg} | {ratio} |")
    return "\n".join(out) + "\n"


def mfma_table(mfma_db: str, trace_db: str, min_calls: int) -> list:
    m = _per_kernel(mfma_db, ("MfmaUtil", "SQ_INSTS_VALU_MFMA_MOPS_F16"))
    trace = _trace(trace_db)
    rows = []
    for key, d in m.items():
        mops = _mean(d.get("SQ_INSTS_VALU_MFMA_MOPS_F16", []))
        durs = trace.get(key, [])
        if not mops or len(durs) < min_calls:
            continue
        flops = mops * 512.0
        us = _mean(durs)
        rows.append({"kernel": key[0], "grid": key[1], "calls": len(durs), "avg_us": round(us, 3),
                     "mfma_util_pct": round(_mean(d.get("MfmaUtil", [])), 2),
                     "mfma_f16_flops": int(flops),
                     "achieved_tflops": round(flops / (us * 1e6), 2)})
    rows.sort(key=lambda x: -x["avg_us"] * x["calls"])
    return rows


STALL_COUNTERS = (
    "SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_ANY",
    "SQ_ACTIVE_INST_VMEM", "SQ_INSTS_VMEM_RD", "SQ_INSTS_VALU", "SQ_ACTIVE_INST_VALU",
    "SQ_ACTIVE_INST_LDS", "SQ_INSTS_LDS", "SQ_INSTS_SMEM", "SQ_BUSY_CU_CYCLES",
    "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_MFMA", "GRBM_GUI_ACTIVE",
    "VmemLatency", "MeanOccupancyPerCU", "MeanOccupancyPerActiveCU",
    "TA_TA_BUSY_sum", "TA_ADDR_STALLED_BY_TC_CYCLES_sum",
    "TCP_TCC_READ_REQ_LATENCY_sum", "TCP_TCC_READ_REQ_sum",
    "TCP_UTCL1_TRANSLATION_MISS_sum", "TCP_UTCL1_TRANSLATION_HIT_sum")


def stall_table(dbs: list, trace_db: str, kernels: list, min_calls: int) -> list:
    """Mean of every stall counter per (kernel, grid) whose short name contains
    one of `kernels`, merged over the pass databases, plus per-wave ratios:
    SQ_WAIT_ANY / SQ_WAVES (cycles a wave spends waiting on a counter),
    SQ_ACTIVE_INST_ANY / SQ_WAVES (cycles it issues), and the average
    TCP-to-L2 read latency (TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ)."""
    merged = collections.defaultdict(dict)
    for db in dbs:
        for key, d in _per_kernel(db, STALL_COUNTERS).items():
            for cname, vals in d.items():
                merged[key][cname] = _mean(vals)
    trace = _trace(trace_db)
    rows = []
    for key, counters in merged.items():
        name, grid = key
        durs = trace.get(key, [])
        if not any(k in name for k in kernels) or len(durs) < min_calls:
            continue
        row = {"kernel": name, "grid": grid, "calls": len(durs), "avg_us": round(_mean(durs), 3)}
        row.update({c: round(v, 3) for c, v in sorted(counters.items())})
        waves = counters.get("SQ_WAVES")
        if waves:
            for c, label in (("SQ_WAIT_ANY", "wait_any_per_wave"),
                             ("SQ_WAIT_INST_ANY", "wait_inst_any_per_wave"),
                             ("SQ_ACTIVE_INST_ANY", "active_inst_any_per_wave"),
                             ("SQ_ACTIVE_INST_VMEM", "active_inst_vmem_per_wave"),
                             ("SQ_INSTS_VMEM_RD", "vmem_rd_insts_per_wave"),
                             ("SQ_INSTS_VALU", "valu_insts_per_wave")):
                if c in counters:
                    row[label] = round(counters[c] / waves, 2)
        req = counters.get("TCP_TCC_READ_REQ_sum")
        if req:
            row["tcp_l2_read_latency_cycles"] = round(
                counters.get("TCP_TCC_READ_REQ_LATENCY_sum", 0.0) / req, 1)
        hit = counters.get("TCP_UTCL1_TRANSLATION_HIT_sum")
        miss = counters.get("TCP_UTCL1_TRANSLATION_MISS_sum")
        if hit is not None and miss is not None and hit + miss:
            row["utcl1_miss_pct"] = round(100.0 * miss / (hit + miss), 2)
        rows.append(row)
    rows.sort(key=lambda x: -x["avg_us"] * x["calls"])
    return rows


C4_WORKLOAD = ("C4 paged GQA decode attention: 16 requests, 32 q / 8 kv heads x 128, pages of "
               "16, lengths U[65, 4096] (seed 403), 2 pools x 3 disjoint block-table sets")


def c4_record(traffic_json: str, stalls_json: str, command: str) -> dict:
    """The attention kernel and the gather probe of the C4 rotation: traffic
    (bytes per launch, L2 hit rate) and stall counters, one entry each, and
    the probe-over-attention ratios the account of the gap rests on."""
    with open(traffic_json) as f:
        traffic_rows = json.load(f)
    with open(stalls_json) as f:
        stall_rows = json.load(f)["kernels"]

    def pick(rows, name):
        found = [r for r in rows if r["kernel"].startswith(name)]
        if not found:
            raise SystemExit(f"{name}: no row")
        return max(found, key=lambda r: r["calls"] * r["avg_us"])

    out = {"workload": C4_WORKLOAD, "command": command, "scales": traffic_rows["scales"]}
    for key, name in (("attention_kernel", "attn_mfma_kernel<4, 1, 4>"),
                      ("gather_probe", "gather_probe_kernel")):
        out[key] = {"traffic": pick(traffic_rows["kernels"], name),
                    "stalls": pick(stall_rows, name)}
    att, probe = out["attention_kernel"]["stalls"], out["gather_probe"]["stalls"]
    ratios = {}
    for field in ("avg_us", "MeanOccupancyPerCU", "VmemLatency", "TA_ADDR_STALLED_BY_TC_CYCLES_sum",
                  "TA_TA_BUSY_sum", "SQ_INSTS_VALU", "SQ_WAIT_ANY"):
        if field in att and field in probe and probe[field]:
            ratios[field] = round(att[field] / probe[field], 3)
    out["attention_over_probe"] = ratios
    out["notes"] = {
        "algorithmic_bytes": "sum of lengths x 8 kv heads x 128 x 2 B x (K and V) + 4 B per "
                             "block-table entry + q and out (fp16)",
        "ea_read_bytes": "32/64/128 B x TCC_EA0_RDREQ_32B/64B/128B per dispatch",
        "MeanOccupancyPerCU": "resident waves per CU averaged over the dispatch",
        "TA_ADDR_STALLED_BY_TC_CYCLES_sum": "texture-addresser cycles stalled by the vector L1, "
                                            "summed over CUs"}
    return out


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
    t.add_argument("--workload", default="")
    t.add_argument("--batch", type=int, default=1)
    t.add_argument("--out")
    b = sub.add_parser("table")
    b.add_argument("--fetch", required=True)
    b.add_argument("--write", required=True)
    b.add_argument("--rdreq", required=True)
    b.add_argument("--trace", required=True)
    b.add_argument("--hit")
    b.add_argument("--copy-bytes", type=int, required=True)
    b.add_argument("--min-calls", type=int, default=2)
    b.add_argument("--algorithmic", action="append",
                   help="name_substring[@grid]=bytes (repeatable)")
    b.add_argument("--title", required=True)
    b.add_argument("--command", required=True)
    b.add_argument("--md")
    b.add_argument("--json")
    m = sub.add_parser("mfma")
    m.add_argument("--db", required=True)
    m.add_argument("--trace", required=True)
    m.add_argument("--min-calls", type=int, default=2)
    m.add_argument("--command", default="")
    m.add_argument("--json")
    st = sub.add_parser("stalls")
    st.add_argument("--db", action="append", required=True, help="pass database (repeatable)")
    st.add_argument("--trace", required=True)
    st.add_argument("--kernel", action="append", required=True,
                    help="short-name substring (repeatable)")
    st.add_argument("--min-calls", type=int, default=2)
    st.add_argument("--command", default="")
    st.add_argument("--workload", default="")
    st.add_argument("--json")
    c = sub.add_parser("c4")
    c.add_argument("--traffic", required=True, help="traffic.json of the extra workload")
    c.add_argument("--stalls", required=True, help="stalls.json of the stalls workload")
    c.add_argument("--command", required=True)
    c.add_argument("--json")
    a = ap.parse_args(argv)
    if a.cmd == "c4":
        text = json.dumps(c4_record(a.traffic, a.stalls, a.command), indent=1) + "\n"
        if a.json:
            with open(a.json, "w") as f:
                f.write(text)
        sys.stdout.write(text)
        return 0
    if a.cmd == "stalls":
        rows = stall_table(a.db, a.trace, a.kernel, a.min_calls)
        text = json.dumps({"workload": a.workload, "command": a.command, "kernels": rows},
                          indent=1) + "\n"
        if a.json:
            with open(a.json, "w") as f:
                f.write(text)
        sys.stdout.write(text)
        return 0
    if a.cmd == "table":
        rows = traffic_table(a.fetch, a.write, a.rdreq, a.trace, a.copy_bytes, a.min_calls,
                             a.algorithmic, a.hit)
        text = table_markdown(rows, a.title, a.command)
        if a.md:
            with open(a.md, "w") as f:
                f.write(text)
        if a.json:
            with open(a.json, "w") as f:
                json.dump({"command": a.command, "scales": rows[0], "kernels": rows[1:]}, f,
                          indent=1)
                f.write("\n")
        sys.stdout.write(text)
        return 0
    if a.cmd == "mfma":
        rows = mfma_table(a.db, a.trace, a.min_calls)
        text = json.dumps({"command": a.command, "peak_tflops_f16": 2500.0, "kernels": rows},
                          indent=1) + "\n"
        if a.json:
            with open(a.json, "w") as f:
                f.write(text)
        sys.stdout.write(text)
        return 0
    if a.cmd == "summary":
        sys.stdout.write(kernel_summary(a.db, a.title, a.command))
        return 0
    result = traffic(a.fetch, a.write, a.kernel, a.template, a.copy_bytes, a.algorithmic)
    result = {"workload": a.workload, "batch": a.batch, **result} if a.workload else result
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
