"""Per-wave timeline of the C4 paged (or C3, or batch-16 decode) attention kernel (MI355X).

Runs bench.py's C4 workload (16 requests, 32 query / 8 kv heads of 128,
16-position pages, lengths U[65, 4096], 6 rotating block-table sets), or with
--workload c3 its C3 workload (one request, 32 heads of 128, L = 4095 + 1 of a
4096 capacity, 8 rotating K/V copies), or with --workload b16 the attention of
the batch-16 7B decode step (16 requests, 32 heads of 128, 16-position pages
of a 1024 capacity, the C5 prompt lengths + 64: one 8-wave block per
(request, head)), through
the library built with TMC_ATTN_TIMELINE=1 (libtmc_hip_timeline.so), reads
the per-wave timestamps of the last launch (tmc_attention_timeline; slot
layout beside the switch in csrc/attention.hip) and reduces them to:

  - the phases of a wave: entry to its first step (length, block table),
    per step the wait for its K/V loads and its arithmetic, the cross-wave
    merge and partial write, the split merge;
  - the launch in 1 us bins: K/V bytes arriving (GB/s), bytes in flight,
    waves computing, waves alive;
  - the placement: waves per CU (HW_ID / XCC_ID) against the time the CU's
    last wave ends.

The timed figure of the plain library is printed beside it: the timeline
build waits for each step's loads before stamping it, which costs about 10%.

Usage (repo root, GPU box):
  python3 aicompiler-test_amd/attention_timeline.py [--workload c3|b16] --json OUT.json --md OUT.md
"""
from __future__ import annotations

import argparse
import collections
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
EVENTS = 48  # slots per wave (kTimelineEvents)
MAX_WAVES = 8192
STEPS = 12  # steps recorded per wave
WORKLOADS = {
    "c4": ("C4 paged GQA decode attention: 16 requests, 32 q / 8 kv heads x 128, pages of 16, "
           "lengths U[65, 4096] (seed 403), 2 pools x 3 disjoint block-table sets"),
    "c3": ("C3 contiguous decode attention: 1 request, 32 heads x 128, L = 4096 of a 4096 "
           "capacity, 8 rotating K/V copies"),
    "b16": ("Batch-16 decode attention of the 7B step: 16 requests, 32 heads x 128, pages of 16, "
            "capacity 1024, lengths = the C5 prompt lengths (U[32, 512], seed 502) + 64, "
            "2 pools x 3 disjoint block-table sets")}


def c4_setup(tmc, torch):
    """bench.py's C4 rotation: returns (launch(i, lib), K/V bytes per launch)."""
    f16 = torch.float16
    d, batch, qh, kvh, p, pages, max_pages = 128, 16, 32, 8, 16, 8192, 256
    lengths = np.random.default_rng(403).integers(64, 4096, size=batch) + 1
    need = (lengths + p - 1) // p
    sets, pools = [], []
    for pool in range(2):
        perm = np.random.default_rng(404 + pool).permutation(pages).astype(np.int32)
        kp = torch.empty((pages, kvh, p, d), dtype=f16, device="cuda")
        vp = torch.empty((pages, kvh, p, d), dtype=f16, device="cuda")
        tmc.fill_normal(kp, 401 + 7 * pool)
        tmc.fill_normal(vp, 402 + 7 * pool)
        pools.append((kp, vp))
        cursor = 0
        for _ in range(3):
            t = np.full((batch, max_pages), -1, np.int32)
            for i in range(batch):
                t[i, :need[i]] = perm[cursor:cursor + need[i]]
                cursor += need[i]
            sets.append((pool, torch.from_numpy(t).cuda()))
    q = torch.empty((batch, qh * d), dtype=f16, device="cuda")
    tmc.fill_normal(q, 405)
    out = torch.empty((batch, qh * d), dtype=f16, device="cuda")
    valid = torch.from_numpy(lengths.astype(np.int32)).cuda()
    active = torch.tensor([batch], dtype=torch.int32, device="cuda")
    ws_bytes = tmc.attention_workspace_bytes(batch, qh, kvh, d, max_pages * p)
    ws = torch.zeros(max(ws_bytes // 4, 1), dtype=torch.float32, device="cuda")

    def launch(i: int) -> None:
        pool, table = sets[i % len(sets)]
        kp, vp = pools[pool]
        tmc.paged_decode_attention(q, kp, vp, valid, table, active, out, batch, qh, kvh, d, p,
                                   max_pages, kvh * p * d, p * d, ws)

    return launch, int(lengths.sum()) * kvh * d * 2 * 2


def b16_setup(tmc, torch):
    """The batch-16 decode step's paged MHA attention at C5's prompt lengths
    plus 64 decoded tokens: returns (launch(i), K/V bytes per launch)."""
    f16 = torch.float16
    d, batch, heads, p, cap = 128, 16, 32, 16, 1024
    max_pages = cap // p
    rng = np.random.default_rng(502)
    lengths = np.array([len(rng.integers(0, 32000, rng.integers(32, 513))) for _ in range(batch)])
    lengths = lengths + 64
    need = (lengths + p - 1) // p
    pages = 3 * int(need.sum())
    sets, pools = [], []
    for pool in range(2):
        perm = np.random.default_rng(504 + pool).permutation(pages).astype(np.int32)
        kp = torch.empty((pages, heads, p, d), dtype=f16, device="cuda")
        vp = torch.empty((pages, heads, p, d), dtype=f16, device="cuda")
        tmc.fill_normal(kp, 501 + 7 * pool)
        tmc.fill_normal(vp, 502 + 7 * pool)
        pools.append((kp, vp))
        cursor = 0
        for _ in range(3):
            t = np.full((batch, max_pages), -1, np.int32)
            for i in range(batch):
                t[i, :need[i]] = perm[cursor:cursor + need[i]]
                cursor += need[i]
            sets.append((pool, torch.from_numpy(t).cuda()))
    q = torch.empty((batch, heads * d), dtype=f16, device="cuda")
    tmc.fill_normal(q, 505)
    out = torch.empty((batch, heads * d), dtype=f16, device="cuda")
    valid = torch.from_numpy(lengths.astype(np.int32)).cuda()
    active = torch.tensor([batch], dtype=torch.int32, device="cuda")
    ws_bytes = tmc.attention_workspace_bytes(batch, heads, heads, d, cap)
    ws = torch.zeros(max(ws_bytes // 4, 1), dtype=torch.float32, device="cuda")

    def launch(i: int) -> None:
        pool, table = sets[i % len(sets)]
        kp, vp = pools[pool]
        tmc.paged_decode_attention(q, kp, vp, valid, table, active, out, batch, heads, heads, d,
                                   p, max_pages, heads * p * d, p * d, ws)

    return launch, int(lengths.sum()) * heads * d * 2 * 2


def c3_setup(tmc, torch):
    """bench.py's C3 rotation (extra_measurements): returns (launch(i), K/V bytes)."""
    f16 = torch.float16
    heads, d, cap, copies, length = 32, 128, 4096, 8, 4096
    ks = [torch.empty((1, heads, cap, d), dtype=f16, device="cuda") for _ in range(copies)]
    vs = [torch.empty_like(ks[0]) for _ in range(copies)]
    for c in range(copies):
        tmc.fill_normal(ks[c], 301 + 10 * c)
        tmc.fill_normal(vs[c], 302 + 10 * c)
    q = torch.empty((1, heads * d), dtype=f16, device="cuda")
    tmc.fill_normal(q, 303)
    out = torch.empty((1, heads * d), dtype=f16, device="cuda")
    valid = torch.tensor([length], dtype=torch.int32, device="cuda")
    ws_bytes = tmc.attention_workspace_bytes(1, heads, heads, d, cap)
    ws = torch.zeros(max(ws_bytes // 4, 1), dtype=torch.float32, device="cuda")

    def launch(i: int) -> None:
        tmc.decode_attention(q, ks[i % copies], vs[i % copies], valid, out, 1, heads, heads, d,
                             cap, ws)

    return launch, heads * length * d * 2 * 2


def analyse(ev: np.ndarray, step_bytes: int = 16384) -> dict:
    """Reduce the [waves, 48] slots of one launch (see the module doc)."""
    ev = ev[ev[:, 0] > 0]
    steps = ev[:, 8]
    live = ev[(steps > 0) & (steps < 99)]
    base = ev[:, 0].min()
    rt0, rt1 = live[:, 0], live[:, 1]
    clock = np.median((live[:, 7] - live[:, 3]) / np.maximum((rt1 - rt0) * 0.01, 1e-9))
    us = lambda cycles: cycles / clock  # shader clock cycles -> us
    pct = lambda a, qs: [round(float(x), 2) for x in np.percentile(a, qs)]
    out = {"waves": int(len(ev)), "live_waves": int(len(live)),
           "no_work_waves": int((steps == 99).sum()),
           "shader_clock_mhz": round(float(clock), 1),
           "span_us": round(float((rt1.max() - base) / 100.0), 2),
           "entry_to_first_step_us_p10_50_90": pct(us(live[:, 4] - live[:, 3]), [10, 50, 90]),
           "entry_to_unit_known_us_p10_50_90": pct(us(live[:, 9] - live[:, 3]), [10, 50, 90]),
           "wave_end_us_p10_50_90_max": pct((rt1 - base) / 100.0, [10, 50, 90, 100])}
    per_step = []
    for s in range(STEPS):
        ok = live[:, 8] > s
        if not ok.any():
            break
        e = live[ok]
        per_step.append({"step": s, "waves": int(ok.sum()),
                         "load_wait_us_p10_50_90": pct(us(e[:, 11 + 3 * s] - e[:, 10 + 3 * s]),
                                                       [10, 50, 90]),
                         "arithmetic_us_p10_50_90": pct(us(e[:, 12 + 3 * s] - e[:, 11 + 3 * s]),
                                                        [10, 50, 90])})
    out["steps"] = per_step
    last = np.array([w[12 + 3 * (min(int(w[8]), STEPS) - 1)] for w in live])
    out["last_step_to_loop_exit_us_p10_50_90"] = pct(us(live[:, 5] - last), [10, 50, 90])
    out["block_meet_and_write_us_p10_50_90"] = pct(us(live[:, 6] - live[:, 5]), [10, 50, 90])
    out["split_merge_us_p50_90_99"] = pct(us(live[:, 7] - live[:, 6]), [50, 90, 99])
    # 1 us bins over the launch
    span = int(out["span_us"]) + 1
    arrive = np.zeros(span + 1)
    flight = np.zeros(span + 1)
    busy = np.zeros(span + 1)
    alive = np.zeros(span + 1)
    start = (rt0 - base) / 100.0
    for i, w in enumerate(live):
        alive[int(start[i]):int((rt1[i] - base) / 100.0) + 1] += 1
        for s in range(min(int(w[8]), STEPS)):
            a = start[i] + us(w[10 + 3 * s] - w[3])
            b = start[i] + us(w[11 + 3 * s] - w[3])
            c = start[i] + us(w[12 + 3 * s] - w[3])
            arrive[min(int(b), span)] += step_bytes
            for t in range(int(a), min(int(b), span) + 1):
                flight[t] += step_bytes * max(0.0, min(b, t + 1) - max(a, t))
            for t in range(int(b), min(int(c), span) + 1):
                busy[t] += max(0.0, min(c, t + 1) - max(b, t))
    out["bins_1us"] = [{"t_us": t, "arrive_gbps": round(arrive[t] / 1e3, 0),
                        "in_flight_mb": round(flight[t] / 1e6, 2), "waves_computing":
                        round(busy[t], 1), "waves_alive": int(alive[t])} for t in range(span)]
    # placement: waves per CU (XCC, SE, SH, CU of HW_ID) and the CU's last end
    hw = live[:, 2] & 0xFFFFFFFF
    xcc = live[:, 2] >> 32
    cu = (xcc << 8) | (((hw >> 13) & 7) << 5) | (((hw >> 12) & 1) << 4) | ((hw >> 8) & 15)
    per_cu = collections.Counter(cu.tolist())
    cu_end = collections.defaultdict(float)
    for i in range(len(live)):
        cu_end[int(cu[i])] = max(cu_end[int(cu[i])], float((rt1[i] - base) / 100.0))
    classes = {}
    for c, n in per_cu.items():
        classes.setdefault(n, []).append(cu_end[c])
    out["cus_used"] = len(per_cu)
    out["by_waves_per_cu"] = [{"live_waves_on_cu": n, "cus": len(v),
                               "cu_end_us_p50_max": pct(v, [50, 100])}
                              for n, v in sorted(classes.items())]
    full = live[live[:, 8] == live[:, 8].max()]
    fcu = (((full[:, 2] >> 32) << 8) | ((((full[:, 2] & 0xFFFFFFFF) >> 13) & 7) << 5) |
           ((((full[:, 2] & 0xFFFFFFFF) >> 12) & 1) << 4) | (((full[:, 2] & 0xFFFFFFFF) >> 8) & 15))
    waves_on = np.array([per_cu[int(c)] for c in fcu])
    total = us(full[:, 7] - full[:, 3])
    out["longest_waves"] = {
        "steps": int(live[:, 8].max()), "waves": int(len(full)),
        "lifetime_us_p10_50_90": pct(total, [10, 50, 90]),
        "load_wait_sum_us_p50": pct(sum(us(full[:, 11 + 3 * s] - full[:, 10 + 3 * s])
                                        for s in range(min(int(live[:, 8].max()), STEPS))),
                                    [50])[0],
        "arithmetic_sum_us_p50": pct(sum(us(full[:, 12 + 3 * s] - full[:, 11 + 3 * s])
                                         for s in range(min(int(live[:, 8].max()), STEPS))),
                                     [50])[0],
        "corr_waves_on_cu_lifetime": round(float(np.corrcoef(waves_on, total)[0, 1]), 3)
        if len(set(waves_on.tolist())) > 1 else None}
    return out


def markdown(rec: dict, command: str) -> str:
    a = rec["timeline"]
    lines = [f"# {rec['workload'].split(':')[0]}: per-wave timeline (MI355X)", "",
             "Command (repo root, MI355X box):", "", f"    {command}", "",
             f"Workload: {rec['workload']}.", "",
             f"Plain library: {rec['plain_us']} us per launch (graph-timed); timeline build "
             f"{rec['timeline_us']} us (each step's loads waited for before its stamp).  "
             f"One launch: {a['live_waves']} waves with work, {a['no_work_waves']} without; "
             f"shader clock {a['shader_clock_mhz']} MHz; span {a['span_us']} us.", "",
             f"- entry to first step (length, block table): p10/50/90 "
             f"{a['entry_to_first_step_us_p10_50_90']} us",
             f"- entry to the block knowing its (request, split) unit (the dealing, paged "
             f"blocks): p10/50/90 {a['entry_to_unit_known_us_p10_50_90']} us",
             f"- wave end: p10/50/90/max {a['wave_end_us_p10_50_90_max']} us",
             f"- last step's stamp to the loop exit: p10/50/90 "
             f"{a['last_step_to_loop_exit_us_p10_50_90']} us",
             f"- the block's waves meet (cross-wave sums in LDS, barrier) and write the partial "
             f"or the output: p10/50/90 {a['block_meet_and_write_us_p10_50_90']} us",
             f"- split merge by the row's last block: p50/90/99 "
             f"{a['split_merge_us_p50_90_99']} us",
             f"- CUs used: {a['cus_used']}", "",
             "Stamps are taken in program order, but the compiler may move independent "
             "arithmetic across a stamp, so a step's split between load wait and arithmetic "
             "is approximate; each wave's totals are exact.",
             "",
             "| step | waves | load wait us p10 / p50 / p90 | arithmetic us p10 / p50 / p90 |",
             "|---|---|---|---|"]
    for s in a["steps"]:
        lines.append(f"| {s['step']} | {s['waves']} | {s['load_wait_us_p10_50_90']} | "
                     f"{s['arithmetic_us_p10_50_90']} |")
    lw = a["longest_waves"]
    lines += ["", f"Longest waves ({lw['waves']} waves of {lw['steps']} steps): lifetime "
              f"p10/50/90 {lw['lifetime_us_p10_50_90']} us, of which load waits "
              f"{lw['load_wait_sum_us_p50']} us and arithmetic {lw['arithmetic_sum_us_p50']} us "
              f"(medians); correlation of lifetime with the waves sharing the CU: "
              f"{lw['corr_waves_on_cu_lifetime']}.", "",
              "| waves with work on the CU | CUs | CU's last wave ends, us p50 / max |",
              "|---|---|---|"]
    for c in a["by_waves_per_cu"]:
        lines.append(f"| {c['live_waves_on_cu']} | {c['cus']} | {c['cu_end_us_p50_max']} |")
    lines += ["", "| t (us) | K/V arriving GB/s | in flight MB | waves computing | waves alive |",
              "|---|---|---|---|---|"]
    for b in a["bins_1us"]:
        lines.append(f"| {b['t_us']} | {b['arrive_gbps']:.0f} | {b['in_flight_mb']} | "
                     f"{b['waves_computing']} | {b['waves_alive']} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--json", required=True)
    ap.add_argument("--md", required=True)
    ap.add_argument("--launches", type=int, default=40)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c4")
    args = ap.parse_args(argv)
    sys.path.insert(0, ROOT)
    import torch
    import bench
    tmc = bench.load_tmc()
    setup = {"c3": c3_setup, "c4": c4_setup, "b16": b16_setup}[args.workload]
    launch, _ = setup(tmc, torch)
    plain_us = bench.time_loop(torch, launch, 60) * 1e6
    saved = tmc.lib()
    variant = tmc.open_variant("libtmc_hip_timeline.so")
    tmc._lib = variant
    try:
        timeline_us = bench.time_loop(torch, launch, 60) * 1e6
        for i in range(args.launches):
            launch(i)
        torch.cuda.synchronize()
        buf = np.zeros(MAX_WAVES * EVENTS, dtype=np.uint64)
        tmc.check(variant.tmc_attention_timeline(buf.ctypes.data, MAX_WAVES),
                  "tmc_attention_timeline")
    finally:
        tmc._lib = saved
    ev = buf.astype(np.int64).reshape(MAX_WAVES, EVENTS)
    flag = "" if args.workload == "c4" else f" --workload {args.workload}"
    command = f"python3 aicompiler-test_amd/attention_timeline.py{flag} --json OUT.json --md OUT.md"
    rec = {"workload": WORKLOADS[args.workload], "command": command, "plain_us": round(plain_us, 2),
           "timeline_us": round(timeline_us, 2), "timeline": analyse(ev)}
    with open(args.json, "w") as f:
        json.dump(rec, f, indent=1)
    with open(args.md, "w") as f:
        f.write(markdown(rec, command))
    print(f"[timeline] plain {plain_us:.2f} us, timeline build {timeline_us:.2f} us, "
          f"span {rec['timeline']['span_us']} us", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
