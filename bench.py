"""Benchmark of the gfx950 decode backend on one MI355X.

Headline workload: the fused Llama decode MLP
block at batch 1 — Add+RMSNorm (hidden 4096), gate/up projection with
SiLU*Mul (intermediate 11008), down projection with fp32 output — with fp16
weights ~N(0, 0.02).  One step = one pass of the block over one batch.  At
batch 1 the block runs as the decoder's batch-1 step runs it: two launches,
the gate/up kernel computing the Add+RMSNorm in its prologue, then down.
`value` is the algorithmic HBM bytes of the block per step x steps / wall
time (GB/s), with every input already resident in HBM.  Weights rotate over
several distinct copies so that the 256 MB Infinity Cache cannot serve them.

Printed JSON line extras:
  roofline      the dominant kernel (Add+RMSNorm + gate/up + SiLU*Mul at batch
                1, gate/up + SiLU*Mul above) timed alone with HIP
                events on the launch stream: algorithmic bytes per launch /
                average launch time, against the 8 TB/s HBM peak;
  cpu_baseline  the CPU oracle (oracle/libtmc_oracle.so, a single-threaded
                C restatement of the reference CPU path) on a bounded number
                of whole blocks of the same workload;
  extra         GB/s of the other BASELINE configs (C1 GEMV, C2 at B=8, C3
                contiguous attention at L=4095, C4 paged GQA attention) and
                C5: Llama-7B-shaped decode tokens/s at batch 1 and 16 (random
                fp16 weights ~N(0, 0.02) made on the device, prompts ~U[32,512]
                run through the batched decode graph, then 128 greedy tokens per
                sequence decoded in lock-step and timed), with the CPU oracle's
                decode step timed on a bounded layer sample beside it.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
COPY_PROBE_BYTES = 256 << 20
# Distinct bytes every kernel-level rotation spans (2 x the 256 MB Infinity Cache)
ROTATE_BYTES = 512 << 20
# HBM bytes per launch of the dominant kernel, measured with rocprofv3
# FETCH_SIZE / WRITE_SIZE and scaled by the copy probe (profiling.py traffic)
TRAFFIC_FILE = "profiles/norm_gate_up_traffic.json"
METRIC = "GEMV/paged-attn HBM GB/s (% of peak); decode tokens/s at batch 1 and 16"
HIDDEN, INTER = 4096, 11008


def load_tmc():
    import importlib.util
    name = "aicompiler_test_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg = os.path.join(ROOT, "aicompiler-test_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(pkg, "__init__.py"),
                                                  submodule_search_locations=[pkg])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def mlp_block_bytes(batch: int) -> dict:
    """Algorithmic bytes of each kernel of the block (fp16 = 2 B, fp32 = 4 B):
    Add+RMSNorm, gate/up + SiLU*Mul and down as three kernels (batch > 1 and
    the CPU oracle), and the batch-1 form whose gate/up kernel computes the
    Add+RMSNorm itself (`norm_gate_up`: the normalized row is neither written
    nor read back)."""
    h, i = HIDDEN, INTER
    add_norm = batch * h * 2 * 4 + h * 2          # read h, r; write s, n; gamma
    gate_up = 2 * i * h * 2 + batch * h * 2 + batch * i * 2
    down = i * h * 2 + batch * i * 2 + batch * h * 4
    norm_gate_up = 2 * i * h * 2 + batch * h * 2 * 3 + h * 2 + batch * i * 2  # h, r, s; gamma
    return {"add_rmsnorm": add_norm, "gate_up_silu": gate_up, "down": down,
            "total": add_norm + gate_up + down, "norm_gate_up": norm_gate_up,
            "fused_total": norm_gate_up + down}


def measured_traffic(batch: int):
    """The committed counter measurement of the dominant kernel, when it was
    taken at this batch size (else None)."""
    path = os.path.join(ROOT, TRAFFIC_FILE)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    return data if data.get("batch", 1) == batch else None


class MlpBlock:
    """Device buffers of the C2 block with `copies` rotating weight sets."""

    def __init__(self, tmc, torch, batch: int, copies: int, packed: bool = False):
        self.tmc, self.torch, self.batch, self.copies = tmc, torch, batch, copies
        self.packed = packed
        f16 = torch.float16
        dev = "cuda"
        self.h = torch.empty((batch, HIDDEN), dtype=f16, device=dev)
        self.r = torch.empty((batch, HIDDEN), dtype=f16, device=dev)
        tmc.fill_normal(self.h, 201)
        tmc.fill_normal(self.r, 202)
        self.weights = []
        for c in range(copies):
            gamma = torch.empty(HIDDEN, dtype=f16, device=dev)
            # U(0.5, 1.5) is not needed bit-exactly: gamma ~ 1 + N(0, 0.25) clipped
            tmc.fill_normal(gamma, 203 + 1000 * c, 1.0, 0.25)
            gamma.clamp_(0.5, 1.5)
            wg = torch.empty((INTER, HIDDEN), dtype=f16, device=dev)
            wu = torch.empty((INTER, HIDDEN), dtype=f16, device=dev)
            wd = torch.empty((HIDDEN, INTER), dtype=f16, device=dev)
            tmc.fill_normal(wg, 204 + 1000 * c, 0.0, 0.02)
            tmc.fill_normal(wu, 205 + 1000 * c, 0.0, 0.02)
            tmc.fill_normal(wd, 206 + 1000 * c, 0.0, 0.02)
            if packed:  # the batch > 1 layout, packed once outside any timed region
                wg, wu, wd = tmc.pack_weights(wg), tmc.pack_weights(wu), tmc.pack_weights(wd)
            self.weights.append((gamma, wg, wu, wd))
        self.s = torch.empty((batch, HIDDEN), dtype=f16, device=dev)
        rows16 = (batch + 15) // 16 * 16  # packed activations fill whole 16-row passes
        self.n = torch.empty((rows16 if packed else batch, HIDDEN), dtype=f16, device=dev)
        self.g = torch.empty((rows16 if packed else batch, INTER), dtype=f16, device=dev)
        self.y = torch.empty((batch, HIDDEN), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()

    def step(self, i: int) -> None:
        gamma, wg, wu, wd = self.weights[i % self.copies]
        t = self.tmc
        if self.packed:  # activations between the kernels in fragment order
            b = self.batch
            t.add_rmsnorm_ex(self.h, self.r, gamma, self.s, self.n, 1e-6, t.Y_PACKED)
            t.gate_up_silu_packed_ex(self.n, wg, wu, self.g, b, HIDDEN, INTER,
                                     t.X_PACKED | t.Y_PACKED)
            t.gemm_packed_ex(self.g, wd, self.y, b, INTER, HIDDEN, t.X_PACKED)
        else:
            t.add_rmsnorm(self.h, self.r, gamma, self.s, self.n, 1e-6)
            t.gate_up_silu(self.n, wg, wu, self.g)
            t.gemv(self.g, wd, self.y)


def build_sequences(tmc, rt, block):
    """Prepared executions of the block for every weight copy, captured as one
    HIP-graph sequence, plus a sequence of the gate/up kernel alone.  Batch 1
    runs the decoder's batch-1 form: gate/up + SiLU*Mul with the Add+RMSNorm
    in its prologue (the sum written, the normalized row kept in registers),
    then down; above batch 1 the norm is its own kernel."""
    b = block.batch
    k_down = rt.resolve(f"decode_gemv?batch={b}&in={INTER}&out={HIDDEN}&out_dtype=f32")
    h, r, s, n = rt.wrap(block.h), rt.wrap(block.r), rt.wrap(block.s), rt.wrap(block.n)
    g, y = rt.wrap(block.g), rt.wrap(block.y)
    execs, gates = [], []
    if b == 1:
        k_fused = rt.resolve(f"add_rmsnorm_gate_up_silu?in={HIDDEN}&out={INTER}&eps=1e-06")
        for gamma, wg, wu, wd in block.weights:
            gm, wgb, wub, wdb = rt.wrap(gamma), rt.wrap(wg), rt.wrap(wu), rt.wrap(wd)
            gate = rt.prepare(k_fused, [h, r, gm, wgb, wub], [s, g])
            execs.append(gate)
            gates.append(gate)
            execs.append(rt.prepare(k_down, [g, wdb], [y]))
        return rt.sequence(execs), execs, rt.sequence(gates)
    k_norm = rt.resolve(f"add_rmsnorm?rows={b}&width={HIDDEN}&eps=1e-06&dtype=f16")
    k_gate = rt.resolve(f"gate_up_silu?batch={b}&hidden={HIDDEN}&inter={INTER}")
    for gamma, wg, wu, wd in block.weights:
        gm, wgb, wub, wdb = rt.wrap(gamma), rt.wrap(wg), rt.wrap(wu), rt.wrap(wd)
        execs.append(rt.prepare(k_norm, [h, r, gm], [s, n]))
        gate = rt.prepare(k_gate, [n, wgb, wub], [g])
        execs.append(gate)
        gates.append(gate)
        execs.append(rt.prepare(k_down, [g, wdb], [y]))
    return rt.sequence(execs), execs, rt.sequence(gates)


def copy_probe(tmc, torch) -> None:
    """Three copies of known size (256 MiB read + 256 MiB written): the
    reference dispatches that scale FETCH_SIZE / WRITE_SIZE (and the EA
    request counters) when a command runs under rocprofv3 --pmc
    (aicompiler-test_amd/profiling.py)."""
    src = torch.empty(COPY_PROBE_BYTES // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        tmc.copy_bytes(src, dst, COPY_PROBE_BYTES)
    torch.cuda.synchronize()
    del src, dst


def time_loop(torch, fn, iters: int, replays: int = 5) -> float:
    """Seconds per call of fn(i): `iters` calls captured once into a CUDA (HIP)
    graph on a side stream, then the graph replayed `replays` times between
    two events, so host launch cost stays out of the figure."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(iters):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / 1000.0 / (iters * replays)


def host_cpu() -> dict:
    """The host the CPU baseline ran on: model name, x86 family / model /
    stepping (the GPU boxes' KVM guests report the model name only as "AMD
    EPYC"; family 26 is Zen 5), hypervisor flag and logical CPU count."""
    fields = {"model name": "unknown", "cpu family": "", "model": "", "stepping": ""}
    hypervisor = False
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, value = line.partition(":")
                key = key.strip()
                if key in fields and fields[key] in ("", "unknown"):
                    fields[key] = value.strip()
                if key == "flags":
                    hypervisor = "hypervisor" in value.split()
                if key == "" and fields["model name"] != "unknown":
                    break
    except OSError:
        pass
    return {"cpu_model": fields["model name"],
            "cpu_family_model_stepping": f"{fields['cpu family']}/{fields['model']}/"
                                         f"{fields['stepping']}",
            "virtualized": hypervisor, "nproc": os.cpu_count()}


def cpu_baseline(block: MlpBlock, seconds: float) -> dict:
    """Whole C2 blocks on the CPU oracle (single thread) with the GPU's copy-0 data."""
    import numpy as np
    from oracle import oracle as orc
    orc.build()
    gamma, wg, wu, wd = block.weights[0]
    as_bits = lambda t: t.detach().cpu().contiguous().numpy().view(np.uint16)  # noqa: E731
    h, r, g16 = as_bits(block.h), as_bits(block.r), as_bits(gamma)
    wg16, wu16, wd16 = as_bits(wg), as_bits(wu), as_bits(wd)
    done, elapsed = 0, 0.0
    t0 = time.perf_counter()
    while done == 0 or elapsed < seconds:
        _, n = orc.add_rmsnorm(h, r, g16, orc.F16, 1e-6)
        n16 = orc.f16(n.astype(np.float32))  # storeValue: float cast, then fp16 (ties away)
        gated = orc.gated_mlp(n16, wg16, wu16, orc.F16)
        orc.linear(orc.f16(gated.astype(np.float32)), wd16, orc.F16)
        done += 1
        elapsed = time.perf_counter() - t0
    total = mlp_block_bytes(block.batch)["total"] * done
    return {"value": round(total / elapsed / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{done} whole C2 blocks (B={block.batch}) on oracle/libtmc_oracle.so, "
                      f"{elapsed:.1f} s, 1 thread", **host_cpu()}


def extra_measurements(tmc, torch, iters: int) -> dict:
    import numpy as np
    out = {}
    f16 = torch.float16
    # Every rotation below spans at least ROTATE_BYTES of distinct buffers,
    # twice the 256 MB Infinity Cache, so no timed launch can be served from it.
    # C1: GEMV fp16 W[4096,4096] -> fp32 y, 16 rotating weight copies (512 MiB)
    c1_copies = -(-ROTATE_BYTES // (4096 * 4096 * 2))
    ws = [torch.empty((4096, 4096), dtype=f16, device="cuda") for _ in range(c1_copies)]
    for c, w in enumerate(ws):
        tmc.fill_normal(w, 103 + c, 0.0, 0.02)
    x = torch.empty((1, 4096), dtype=f16, device="cuda")
    tmc.fill_normal(x, 101)
    y = torch.empty((1, 4096), dtype=torch.float32, device="cuda")
    sec = time_loop(torch, lambda i: tmc.gemv(x, ws[i % c1_copies], y), iters)
    gemv_bytes = 4096 * 4096 * 2 + 4096 * 2 + 4096 * 4
    out["c1_gemv_4096x4096_gbps"] = round(gemv_bytes / sec / 1e9, 1)
    out["c1_gemv_us"] = round(sec * 1e6, 2)
    # the floor of one launch that reads the same 32 MiB once: the read-only
    # probe over the same rotation
    sink = torch.zeros(1, dtype=torch.float32, device="cuda")
    floor = time_loop(torch, lambda i: tmc.read_probe(ws[i % c1_copies], 4096 * 4096 * 2, sink),
                      iters)
    out["c1_read_floor_us"] = round(floor * 1e6, 2)
    out["c1_frac_of_read_floor"] = round(floor / sec, 3)
    del ws
    # C2 at B=8: the batch > 1 path runs on fragment-packed weights; the
    # row-major MFMA kernel is timed beside it
    blk = MlpBlock(tmc, torch, 8, 4, packed=True)
    sec = time_loop(torch, blk.step, iters)
    out["c2_mlp_block_b8_gbps"] = round(mlp_block_bytes(8)["total"] / sec / 1e9, 1)
    out["c2_mlp_block_b8_us"] = round(sec * 1e6, 2)
    del blk
    blk = MlpBlock(tmc, torch, 8, 4)
    sec = time_loop(torch, blk.step, iters)
    out["c2_mlp_block_b8_rowmajor_gbps"] = round(mlp_block_bytes(8)["total"] / sec / 1e9, 1)
    del blk
    # C3: contiguous attention, 32 heads x 128, capacity 4096, valid 4096 (L=4095 + 1)
    heads, d, cap = 32, 128, 4096
    copies = -(-ROTATE_BYTES // (2 * heads * cap * d * 2))  # 8 K/V pairs of 64 MiB
    ks = [torch.empty((1, heads, cap, d), dtype=f16, device="cuda") for _ in range(copies)]
    vs = [torch.empty((1, heads, cap, d), dtype=f16, device="cuda") for _ in range(copies)]
    for c in range(copies):
        tmc.fill_normal(ks[c], 301 + 10 * c)
        tmc.fill_normal(vs[c], 302 + 10 * c)
    q = torch.empty((1, heads * d), dtype=f16, device="cuda")
    tmc.fill_normal(q, 303)
    o = torch.empty((1, heads * d), dtype=f16, device="cuda")
    valid = torch.tensor([4096], dtype=torch.int32, device="cuda")
    wsb = tmc.attention_workspace_bytes(1, heads, heads, d, cap)
    wsp = torch.zeros(max(wsb // 4, 1), dtype=torch.float32, device="cuda")
    sec = time_loop(torch, lambda i: tmc.decode_attention(q, ks[i % copies], vs[i % copies], valid,
                                                          o, 1, heads, heads, d, cap, wsp), iters)
    c3_bytes = 2 * heads * 4096 * d * 2 + 2 * heads * d * 2
    out["c3_attention_L4095_gbps"] = round(c3_bytes / sec / 1e9, 1)
    del ks, vs
    # C4: paged GQA attention, 16 requests, 32 q / 8 kv heads, pages of 16.
    # Two pools of 8192 pages (K and V, 512 MiB each pool); each holds 3
    # disjoint table sets, so the rotation reads 6 x 148 MB of distinct pages.
    batch, qh, kvh, p, pages, max_pages = 16, 32, 8, 16, 8192, 256
    lengths = np.random.default_rng(403).integers(64, 4096, size=batch) + 1
    need = (lengths + p - 1) // p
    sets = []
    pools = []
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
    qd = torch.empty((batch, qh * d), dtype=f16, device="cuda")
    tmc.fill_normal(qd, 405)
    od = torch.empty((batch, qh * d), dtype=f16, device="cuda")
    vl = torch.from_numpy(lengths.astype(np.int32)).cuda()
    active = torch.tensor([batch], dtype=torch.int32, device="cuda")
    wsb = tmc.attention_workspace_bytes(batch, qh, kvh, d, max_pages * p)
    wsp = torch.zeros(max(wsb // 4, 1), dtype=torch.float32, device="cuda")

    def c4(i):
        pool, table = sets[i % len(sets)]
        kp, vp = pools[pool]
        tmc.paged_decode_attention(qd, kp, vp, vl, table, active, od, batch, qh, kvh, d, p,
                                   max_pages, kvh * p * d, p * d, wsp)

    sec = time_loop(torch, c4, iters)
    c4_bytes = int(lengths.sum()) * kvh * d * 2 * 2 + 4 * int(need.sum()) + 2 * batch * qh * d * 2
    out["c4_paged_gqa_attention_gbps"] = round(c4_bytes / sec / 1e9, 1)
    out["c4_paged_gqa_attention_us"] = round(sec * 1e6, 2)
    out["c4_bytes"] = c4_bytes
    # The same K/V bytes through the same tables with nothing but loads
    # (tmc_paged_gather_probe): the ceiling of the gather itself.
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def gather(i):
        pool, table = sets[i % len(sets)]
        kp, vp = pools[pool]
        tmc.paged_gather_probe(kp, vp, vl, table, batch, kvh, d, p, max_pages, kvh * p * d, p * d,
                               sink)

    sec = time_loop(torch, gather, iters)
    kv_bytes = int(lengths.sum()) * kvh * d * 2 * 2
    out["c4_gather_probe_gbps"] = round(kv_bytes / sec / 1e9, 1)
    out["c4_gather_probe_us"] = round(sec * 1e6, 2)
    del pools
    out["rotation_min_bytes"] = ROTATE_BYTES
    # rocprofv3 counter tables behind these figures (per-kernel HBM bytes
    # from FETCH_SIZE / WRITE_SIZE and the EA request counters, L2 hit rate,
    # MfmaUtil), made by aicompiler-test_amd/profile_counters.sh
    out["counter_files"] = {
        "c1_c2b8_c3_c4": "profiles/c1_c4_kernels_traffic.md",
        "c4_attention": "profiles/attention_c4_counters.json",
        "c1_c4_stalls": "profiles/c1_c4_stall_counters.json",
        "c2_b8_mfma": "profiles/c2_b8_mfma_utilisation.json",
        "c5_decode": "profiles/c5_decode_prefill_traffic.md",
        "c5_mfma": "profiles/c5_mfma_utilisation.json"}
    return out


C5 = dict(layers=32, hidden=4096, heads=32, head_dim=128, intermediate=11008, vocabulary=32000,
          capacity=1024, epsilon=1e-6, page_size=16, decode_tokens=128, prefill_chunk=1024)
# Chunked prefill of one long prompt on the same 7B shape (capacity 4096).
PREFILL = dict(capacity=4096, prompts=(4095, 512), chunks=(512, 2048))


def c5_plan(host, capacity=None):
    plan = host.DecoderLLMPlan()
    att = host.KVCachePlan()
    att.heads, att.head_dimension = C5["heads"], C5["head_dim"]
    att.capacity = capacity or C5["capacity"]
    att.dtype = host.DType.Float16
    plan.attention = att
    plan.layer_count, plan.intermediate_size = C5["layers"], C5["intermediate"]
    plan.vocabulary_size, plan.rms_norm_epsilon = C5["vocabulary"], C5["epsilon"]
    return plan


def c5_prompts(batch: int):
    import numpy as np
    rng = np.random.default_rng(502)
    return [list(map(int, rng.integers(0, C5["vocabulary"], rng.integers(32, 513))))
            for _ in range(batch)]


def c5_gpu(tmc) -> dict:
    """Decode tokens/s of the 7B-shaped model at batch 1 and 16 (C++ host
    layer: graph-captured batched decode over paged KV pools).  Prompts run
    through the chunked prefill executor first (its own timed phase)."""
    host = tmc.host()
    rt = host.HipRuntime()
    model = host.create_synthetic_model_resources(rt, c5_plan(host), 501)
    out = {"model_bytes": int(model.storage_bytes)}
    for batch in (1, 16):
        r = host.measure_decode_throughput(rt, model, c5_prompts(batch), C5["decode_tokens"],
                                           C5["page_size"], False, False, C5["prefill_chunk"])
        if not r["passed"]:
            raise RuntimeError(f"C5 batch {batch}: {r['error']}")
        steps = r["decode_steps"]
        out[f"b{batch}_tokens_per_s"] = round(r["tokens_per_second"], 1)
        out[f"b{batch}_ms_per_step"] = round(r["decode_phase_us"] / steps / 1e3, 4)
        # bytes a step must read: every weight except the embedding table (B
        # rows of it), plus the K/V of every attended position
        weights = model.storage_bytes - C5["vocabulary"] * C5["hidden"] * 2
        out[f"b{batch}_weight_and_kv_gbps"] = round(
            (weights * steps + r["kv_bytes_read"]) / (r["decode_phase_us"] * 1e3), 1)
        out[f"b{batch}_prompt_tokens"] = sum(len(p) for p in c5_prompts(batch))
        out[f"b{batch}_prompt_ms"] = round(r["prompt_phase_us"] / 1e3, 2)
        out[f"b{batch}_prompt_tokens_per_s"] = round(r["prompt_tokens_per_second"], 1)
        # the token-only LM head tail (partial + final argmax), admitted only
        # at >= 1.05x over the logits tail in two paired rounds
        out[f"b{batch}_token_only"] = {"admitted": r["token_only_admitted"],
                                        "speedup": round(r["token_only_speedup"], 4)}
        print(f"[bench] C5 batch {batch}: {out[f'b{batch}_tokens_per_s']} tokens/s, prompts "
              f"{out[f'b{batch}_prompt_tokens_per_s']} tokens/s", flush=True)
        out[f"b{batch}_serving"] = c5_serving(host, rt, model, batch)
    out["prefill_chunk"] = C5["prefill_chunk"]
    del model
    return out


def c5_serving(host, rt, model, batch: int) -> dict:
    """The same requests through runContinuousBatch (ServingRuntime.cpp:513-930):
    admission with packed chunked prefill, then scheduler-driven batched decode
    ticks with a host round trip per tick (tokens read back, tables updated),
    as a serving loop runs them.  tokens/s over the whole run and over the
    ticks without prompt rows."""
    prompts = c5_prompts(batch)
    specs = []
    for i, prompt in enumerate(prompts):
        spec = host.ServingRequestSpec()
        spec.id = f"r{i}"
        spec.prompt_token_ids = [float(t) for t in prompt]
        spec.decode_token_count = C5["decode_tokens"]
        spec.arrival_step = 0
        specs.append(spec)
    pages = (max(len(p) for p in prompts) + C5["decode_tokens"] + C5["page_size"] - 1) \
        // C5["page_size"]
    config = host.ServingConfig()
    config.page_size = C5["page_size"]
    config.physical_pages_per_layer = max(batch * pages, C5["capacity"] // C5["page_size"])
    config.maximum_batch_size = batch
    config.record_decode_logits = False
    config.record_prefill_logits = False
    config.prefill_chunk_size = C5["prefill_chunk"]
    config.prefill_requests_per_chunk = batch
    r = host.run_continuous_batch(rt, model, specs, config)
    if not r["passed"]:
        raise RuntimeError(f"C5 serving batch {batch}: {r['error']}")
    m = r["metrics"]
    print(f"[bench] C5 serving batch {batch}: {m['decode_phase_tokens_per_second']:.1f} decode "
          f"tokens/s, {m['tokens_per_second']:.1f} over the run", flush=True)
    return {"decode_tokens_per_s": round(m["decode_phase_tokens_per_second"], 1),
            "run_tokens_per_s": round(m["tokens_per_second"], 1),
            "total_ms": round(m["total_time_us"] / 1e3, 2),
            "decoded_tokens": m["decoded_tokens"], "prompt_tokens": m["prompt_tokens"],
            "decode_ticks": m["decode_command_submissions"],
            "prefill_chunks": m["prefill_chunk_submissions"],
            "scheduler_overhead_ms": round(m["scheduler_overhead_us"] / 1e3, 2)}


def prefill_flops(tokens: int) -> float:
    """Prompt FLOPs of the 7B shape: 2 per weight per token for every matrix
    (q.k.v, o, gate, up, down in 32 layers, and the LM head on every row) plus
    causal attention, 4 * D * heads per attended position per layer."""
    h, i, v, layers = C5["hidden"], C5["intermediate"], C5["vocabulary"], C5["layers"]
    weights = layers * (h * 3 * h + h * h + 3 * h * i) + v * h
    attended = tokens * (tokens + 1) / 2
    return 2.0 * weights * tokens + 4.0 * C5["head_dim"] * C5["heads"] * layers * attended


def prefill_gpu(tmc) -> dict:
    """Chunked prefill throughput of the 7B shape: one prompt per run through
    the MFMA prompt GEMMs and the MFMA causal chunk attention; TFLOP/s
    against the 2.5 PFLOP/s dense fp16 peak."""
    host = tmc.host()
    rt = host.HipRuntime()
    model = host.create_synthetic_model_resources(rt, c5_plan(host, PREFILL["capacity"]), 503)
    import numpy as np
    rng = np.random.default_rng(504)
    out = {"capacity": PREFILL["capacity"]}
    for length in PREFILL["prompts"]:
        prompt = [list(map(int, rng.integers(0, C5["vocabulary"], length)))]
        for chunk in PREFILL["chunks"]:
            if chunk > length and chunk != PREFILL["chunks"][0]:
                continue
            r = host.measure_decode_throughput(rt, model, prompt, 1, C5["page_size"], False, False,
                                               chunk)
            if not r["passed"]:
                raise RuntimeError(f"prefill {length}/{chunk}: {r['error']}")
            sec = r["prompt_phase_us"] / 1e6
            key = f"p{length}_c{chunk}"
            out[key + "_ms"] = round(sec * 1e3, 2)
            out[key + "_tokens_per_s"] = round(length / sec, 1)
            out[key + "_tflops"] = round(prefill_flops(length) / sec / 1e12, 1)
            print(f"[bench] prefill {length} tokens, chunk {chunk}: {out[key + '_ms']} ms, "
                  f"{out[key + '_tokens_per_s']} tokens/s", flush=True)
    out["peak_tflops"] = 2500.0
    del model
    return out


def c5_cpu_baseline(steps: int = 2) -> dict:
    """The oracle's decode step (oracle/libtmc_oracle.so, one thread) at the
    C5 shape: `steps` whole decode steps (32 layers, the LM head over every
    row, greedy tokens) at batch 1 and at batch 16, fed back token to token.
    Weight values do not change the oracle's work, so fixed fp16 patterns
    stand in for random weights, and the 32 layers share one layer's arrays
    (the same arithmetic as 32 distinct layers, a fraction of the host
    memory)."""
    import numpy as np
    from oracle import oracle as orc
    orc.build()
    H, I, V, NH, D = C5["hidden"], C5["intermediate"], C5["vocabulary"], C5["heads"], C5["head_dim"]
    L = C5["layers"]
    pattern = np.random.default_rng(0).integers(0x2000, 0x2c00, 4096, dtype=np.uint16)
    pattern[1::2] |= 0x8000
    w = lambda *shape: np.resize(pattern, shape)  # noqa: E731
    one = np.full(H, 0x3C00, np.uint16)
    cap = 64
    pos = np.arange(cap)[:, None]
    freq = 10000.0 ** (-np.arange(0, D, 2) / D)
    layer = dict(input_norm=one, wq=w(H, H), wk=w(H, H), wv=w(H, H), wo=w(H, H), post_norm=one,
                 wg=w(I, H), wu=w(I, H), wd=w(H, I))
    out = {}
    for batch in (1, 16):
        m = dict(embedding=w(V, H), final_norm=one, lm_head=w(V, H),
                 rope_cos=np.cos(pos * freq).astype(np.float32),
                 rope_sin=np.sin(pos * freq).astype(np.float32), layers=[layer] * L)
        cfg = dict(layers=L, hidden=H, heads=NH, head_dim=D, intermediate=I, vocabulary=V,
                   capacity=cap, epsilon=1e-6)
        pages = cap // 16
        kp = [np.zeros(batch * pages * NH * 16 * D, np.uint16) for _ in range(L)]
        vp = [np.zeros_like(p) for p in kp]
        tables = np.zeros((L, batch, pages), np.int32)
        for b in range(batch):
            tables[:, b, :] = b * pages + np.arange(pages)
        tokens = np.arange(batch, dtype=np.int32)
        t0 = time.perf_counter()
        for s in range(steps):
            _, tokens = orc.decoder_step(m, cfg, kp, vp, 16, pages, tables, tokens,
                                         np.full(batch, s + 1, np.int32))
            tokens = np.asarray(tokens, np.int32)
        elapsed = time.perf_counter() - t0
        out[f"b{batch}_tokens_per_s"] = round(batch * steps / elapsed, 5)
        out[f"b{batch}_sample"] = (f"{steps} whole decode steps (32 layers + LM head + argmax, "
                                   f"{batch} row(s)) in {elapsed:.1f} s")
    out["cores"] = 1
    out.update(host_cpu())
    out["kind"] = "port"
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--copies", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the chunked prefill measurement and print its JSON (for profiling)")
    ap.add_argument("--c5-only", action="store_true",
                    help="run only the C5 decode measurement (batch 1 and 16) and print its JSON "
                         "(for profiling)")
    ap.add_argument("--extra-only", action="store_true",
                    help="run only the copy probe and the C1-C4 kernel measurements and print "
                         "their JSON (for profiling)")
    ap.add_argument("--decode-tokens", type=int, default=C5["decode_tokens"],
                    help="greedy decode tokens per sequence in the C5 measurement")
    args = ap.parse_args()
    C5["decode_tokens"] = args.decode_tokens
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1).", file=sys.stderr)
        return 2

    import torch
    tmc = load_tmc()
    tmc.lib()
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_gpu(tmc)}), flush=True)
        return 0
    if args.c5_only:
        copy_probe(tmc, torch)
        print(json.dumps({"c5_decode": c5_gpu(tmc)}), flush=True)
        return 0
    if args.extra_only:
        copy_probe(tmc, torch)
        print(json.dumps({"extra": extra_measurements(tmc, torch, 40)}), flush=True)
        return 0
    block = MlpBlock(tmc, torch, args.batch, args.copies)
    # The timed region replays a HIP graph built by the backend's own
    # PreparedSequence counterpart (tmc_seq_*): one graph holds one step per
    # weight copy, so a replay is `copies` steps.
    rt = tmc.Runtime()
    seq, execs, gate_seq = build_sequences(tmc, rt, block)
    torch.cuda.synchronize()
    print(f"[bench] C2 block B={args.batch}, {args.copies} weight copies; warmup", flush=True)
    replays = max(1, args.steps // args.copies)
    steps = replays * args.copies
    for _ in range(max(1, args.warmup // args.copies)):
        seq.launch()
    rs = rt.torch_stream()
    rs.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        seq.launch()
    rs.synchronize()
    elapsed = time.perf_counter() - t0
    bytes_ = mlp_block_bytes(args.batch)
    fused = args.batch == 1
    block_bytes = bytes_["fused_total"] if fused else bytes_["total"]
    gate_bytes = bytes_["norm_gate_up"] if fused else bytes_["gate_up_silu"]
    value = block_bytes * steps / elapsed / 1e9
    print(f"[bench] timed {steps} steps in {elapsed:.4f} s", flush=True)

    copy_probe(tmc, torch)

    # dominant kernel alone: gate/up + SiLU*Mul over the rotating weight
    # copies, HIP events on the runtime stream around graph replays
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gate_replays = max(1, steps // args.copies)
    gate_seq.launch()
    start.record(rs)
    for _ in range(gate_replays):
        gate_seq.launch()
    stop.record(rs)
    stop.synchronize()
    sec = start.elapsed_time(stop) / 1000.0 / (gate_replays * args.copies)
    achieved = gate_bytes / sec / 1e9
    measured = measured_traffic(args.batch)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": measured["traffic_bytes_per_launch"] if measured else None,
                "kernel": ("gemv_norm_kernel<2,1,2> (Add+RMSNorm + gate/up + SiLU*Mul)" if fused
                           else "gemv_dot_kernel (gate/up + SiLU*Mul)"),
                "bytes_per_launch": gate_bytes, "avg_launch_us": round(sec * 1e6, 3)}
    if measured:
        roofline["traffic_source"] = TRAFFIC_FILE
        roofline["traffic_over_algorithmic"] = measured.get("traffic_over_algorithmic")
    print(f"[bench] {'norm + ' if fused else ''}gate_up_silu {sec * 1e6:.2f} us/launch", flush=True)
    del execs
    steps_reported = steps
    extra = {} if args.no_extra else extra_measurements(tmc, torch, 40)
    print("[bench] extras done", flush=True)
    if not args.no_extra:
        extra["c5_decode"] = c5_gpu(tmc)
        if not args.no_cpu:
            extra["c5_decode"]["cpu_baseline"] = c5_cpu_baseline()
        extra["prefill"] = prefill_gpu(tmc)
    cpu = None if args.no_cpu else cpu_baseline(block, args.cpu_seconds)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": steps_reported, "warmup": args.warmup,
        "ms_per_step": round(elapsed / steps_reported * 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "C2 fused decode MLP block: Add+RMSNorm -> gate/up+SiLU*Mul -> "
                               "down (fp32 out); hidden 4096, intermediate 11008",
                   "batch": args.batch, "weight_copies": args.copies, "accumulate": "f32",
                   "bytes_per_step": block_bytes, "frac_of_hbm_peak":
                       round(value / HBM_PEAK_GBPS, 4)},
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
