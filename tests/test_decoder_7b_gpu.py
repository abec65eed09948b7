"""GPU parity of the decode path at the Llama-7B widths of the C5 workload
(hidden 4096, 32 heads x 128, intermediate 11008, vocabulary 32000, RoPE
theta 10000, fp16 weights ~ N(0, 0.02)) on 2 layers, against the oracle's
decoder step (oracle/tmc_oracle.c tmco_decoder_step, pinned by
test_oracle_decoder.py) on the same weights and tokens.

At these widths the decoder selects kernels the small-shape tests never run
together: 512-thread norms, the two-rows-per-wave GEMV defaults with the
q.k.v + RoPE + append epilogue (batch 1), the one-split 16-wave attention
(capacity 1024) or the split attention with its merge (capacity 4096), and
at batch 16 the packed GEMMs with the RoPE + append epilogue and packed
activations.  Reference behaviour: CompiledDecoderLLM::decode/prefillChunked
(DecoderLLMExecutor.cpp:881-1048) and runContinuousBatch (ServingRuntime.cpp:
513-930).

Tolerances (tests/helpers.py): logits and K/V are fp16-path values (2e-2
absolute, 3e-3 relative RMS); a greedy token may differ from the oracle's
only where the oracle's top two logits are closer than 2e-2.  The oracle
follows the GPU's token sequence, so one near-tie does not end the check."""
import os

import numpy as np
import pytest

from tests.helpers import assert_f16_path
from tests.test_decoder_gpu import OracleRequest, P, _check_token, _workload

pytestmark = pytest.mark.gpu

SHAPE = dict(layers=2, hidden=4096, heads=32, head_dim=128, kv_heads=32, intermediate=11008,
             vocabulary=32000, epsilon=1e-6)
ROPE_ROWS = 4096


def _cfg(capacity):
    return dict(SHAPE, capacity=capacity)


def _oracle_threads():
    return max(1, min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def weights7b(orc):
    """fp16 bit arrays of a 2-layer 7B-width model (seed 5001): matrices
    ~ N(0, 0.02), norm weights ~ U(0.5, 1.5), RoPE tables for 4096 rows."""
    rng = np.random.default_rng(5001)
    H, I, V, D = SHAPE["hidden"], SHAPE["intermediate"], SHAPE["vocabulary"], SHAPE["head_dim"]
    kv = SHAPE["kv_heads"] * D
    f16 = lambda a: orc.f16(np.asarray(a, np.float32))  # noqa: E731

    def w(*shape):
        # N(0, 0.02) by Box-Muller on float32 uniforms (numpy's own normal
        # sampler takes minutes for the 0.7 G values of this model)
        u1 = rng.random(shape, dtype=np.float32)
        u2 = rng.random(shape, dtype=np.float32)
        z = np.sqrt(np.float32(-2.0) * np.log1p(-u1)) * np.cos(np.float32(2 * np.pi) * u2)
        return f16(z * np.float32(0.02))

    layers = [dict(input_norm=f16(rng.uniform(0.5, 1.5, H)), wq=w(H, H), wk=w(kv, H),
                   wv=w(kv, H), wo=w(H, H), post_norm=f16(rng.uniform(0.5, 1.5, H)),
                   wg=w(I, H), wu=w(I, H), wd=w(H, I)) for _ in range(SHAPE["layers"])]
    pos = np.arange(ROPE_ROWS, dtype=np.float64)[:, None]
    freq = 10000.0 ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    print("[7b] host weights ready", flush=True)
    return dict(embedding=w(V, H), final_norm=f16(rng.uniform(0.5, 1.5, H)), lm_head=w(V, H),
                rope_cos=np.cos(pos * freq).astype(np.float32),
                rope_sin=np.sin(pos * freq).astype(np.float32), layers=layers)


class _FastValues:
    """fp16 bits -> float32 values for the upload (IEEE fp16 -> fp32 is
    exact, so numpy's conversion gives the oracle's values)."""

    @staticmethod
    def f16_values(bits):
        return np.ascontiguousarray(bits, np.uint16).view(np.float16).astype(np.float32)


def _at_capacity(m, capacity):
    return dict(m, rope_cos=m["rope_cos"][:capacity], rope_sin=m["rope_sin"][:capacity])


@pytest.fixture(scope="module")
def rt7b(host):
    r = host.HipRuntime()
    assert r.is_available(), r.initialization_error()
    return r


@pytest.fixture(scope="module")
def models7b(host, orc, rt7b, weights7b):
    """Device model resources per capacity, uploaded once."""
    cache = {}

    def get(capacity):
        if capacity not in cache:
            cfg = _cfg(capacity)
            w = _workload(host, _FastValues, cfg, _at_capacity(weights7b, capacity))
            cache[capacity] = (host.create_model_resources(rt7b, w), w.plan)
            del w
            print(f"[7b] model uploaded (capacity {capacity})", flush=True)
        return cache[capacity]

    yield get
    cache.clear()


def _decoder(host, rt, model, plan, chunk):
    w = host.DecoderLLMWorkload()
    w.plan = plan
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    opts.prefill_chunk_size = chunk
    opts.shared_model_resources = model
    dec, log = host.compile_decoder_llm(rt, w, opts)
    return dec, log


def _prompt(seed, lo, hi):
    rng = np.random.default_rng(seed)
    return rng.integers(0, SHAPE["vocabulary"], int(rng.integers(lo, hi + 1)))


@pytest.mark.parametrize("capacity,chunk,lo,hi", [(1024, 128, 32, 512), (4096, 512, 600, 700)])
def test_7b_decoder_batch1_matches_oracle(host, orc, rt7b, weights7b, models7b, capacity, chunk,
                                          lo, hi):
    """Batch 1: a prompt through chunked prefill, then 3 decode steps.
    Capacity 1024 is C5's (one-split attention); at capacity 4096 a row of
    600+ positions is cut into 512-position splits and merged."""
    model, plan = models7b(capacity)
    cfg = _cfg(capacity)
    m = _at_capacity(weights7b, capacity)
    dec, log = _decoder(host, rt7b, model, plan, chunk)
    assert "Chunked prefill stage" in log
    prompt = _prompt(7000 + capacity, lo, hi)
    n, V = len(prompt), SHAPE["vocabulary"]
    print(f"[7b] batch 1 capacity {capacity}: prompt {n} tokens, chunk {chunk}", flush=True)
    res = dec.prefill_chunked([float(t) for t in prompt], True)
    assert res["passed"], res["error"]
    gpu_logits = res["logits"].reshape(n, V)
    tables = [dec.kv_block_table(l) for l in range(SHAPE["layers"])]
    ref = OracleRequest(orc, cfg, m, capacity // P)
    t = np.full((SHAPE["layers"], n, capacity // P), -1, np.int32)
    for l, table in enumerate(tables):
        t[l, :, :len(table)] = table
    orc.set_threads(_oracle_threads())
    try:
        ref_logits, ref_next = orc.decoder_step(m, cfg, ref.k, ref.v, P, capacity // P, t, prompt,
                                                np.arange(1, n + 1))
        assert_f16_path(gpu_logits, ref_logits, f"cap {capacity} prefill logits")
        token = int(res["next_token_ids"][-1])
        _check_token(token, int(ref_next[-1]), ref_logits[-1], f"cap {capacity} first token")
        for step in range(3):
            out = dec.decode([float(token)], True)
            assert out["passed"], out["error"]
            tables = [dec.kv_block_table(l) for l in range(SHAPE["layers"])]
            logits, nxt = ref.step(token, n + step + 1, tables)
            assert_f16_path(out["logits"], logits, f"cap {capacity} decode step {step}")
            _check_token(int(out["next_token_ids"][0]), nxt, logits, f"cap {capacity} step {step}")
            token = int(out["next_token_ids"][0])
    finally:
        orc.set_threads(1)
    length = dec.current_length()
    assert length == n + 3
    kvh, d = SHAPE["kv_heads"], SHAPE["head_dim"]
    for l in range(SHAPE["layers"]):
        table = dec.kv_block_table(l)
        assert_f16_path(dec.read_key_prefix(l).reshape(kvh, length, d),
                        ref.prefix(l, table, length, True), f"cap {capacity} layer {l} keys")
        assert_f16_path(dec.read_value_prefix(l).reshape(kvh, length, d),
                        ref.prefix(l, table, length, False), f"cap {capacity} layer {l} values")


def test_7b_serving_batch16_matches_oracle(host, orc, rt7b, weights7b, models7b):
    """Batch 16 through runContinuousBatch (C5's structure): 16 prompts
    ~ U[32, 512] prefilled in packed chunks at admission, then 3 lock-step
    decode ticks of 16 rows on the packed GEMMs.  The oracle replays every
    request from its prompt with the tokens the GPU generated."""
    capacity, batch, steps = 1024, 16, 3
    model, _ = models7b(capacity)
    cfg = _cfg(capacity)
    m = _at_capacity(weights7b, capacity)
    V = SHAPE["vocabulary"]
    rng = np.random.default_rng(7100)
    prompts = [rng.integers(0, V, int(rng.integers(32, 513))) for _ in range(batch)]
    specs = []
    for i, prompt in enumerate(prompts):
        s = host.ServingRequestSpec()
        s.id = f"r{i}"
        s.prompt_token_ids = [float(t) for t in prompt]
        s.decode_token_count = steps
        s.arrival_step = 0
        specs.append(s)
    per_request = (max(len(p) for p in prompts) + steps + P - 1) // P
    config = host.ServingConfig()
    config.page_size = P
    config.physical_pages_per_layer = batch * per_request
    config.maximum_batch_size = batch
    config.record_decode_logits = True
    config.prefill_chunk_size = 1024
    config.prefill_requests_per_chunk = batch
    print(f"[7b] serving batch {batch}: prompts {[len(p) for p in prompts]}", flush=True)
    result = host.run_continuous_batch(rt7b, model, specs, config)
    assert result["passed"], result["error"]
    metrics = result["metrics"]
    assert metrics["maximum_active_batch_size"] == batch
    assert metrics["preemption_count"] == 0
    outs = result["requests"]
    for spec, out in zip(specs, outs):
        assert out["id"] == spec.id and len(out["generated_token_ids"]) == steps + 1

    # Oracle: every request owns `per_request` pages of one shared pool.  The
    # prompts run in groups of 4 requests, all prompt rows of a group as one
    # step (each request's rows in position order) with each request's last
    # prompt row at the end, so the LM head runs only there.
    max_pages = capacity // P
    pool = batch * per_request * SHAPE["kv_heads"] * P * SHAPE["head_dim"]
    kp = [np.zeros(pool, np.uint16) for _ in range(SHAPE["layers"])]
    vp = [np.zeros(pool, np.uint16) for _ in range(SHAPE["layers"])]
    table = np.full((batch, max_pages), -1, np.int32)
    for r in range(batch):
        table[r, :per_request] = r * per_request + np.arange(per_request)
    orc.set_threads(_oracle_threads())
    try:
        for group in range(0, batch, 4):
            members = range(group, min(group + 4, batch))
            rows = [(r, i) for r in members for i in range(len(prompts[r]) - 1)]
            rows += [(r, len(prompts[r]) - 1) for r in members]
            req = np.array([r for r, _ in rows])
            tokens = np.array([prompts[r][i] for r, i in rows], np.int32)
            lengths = np.array([i + 1 for _, i in rows], np.int32)
            tables = np.broadcast_to(table[req], (SHAPE["layers"], len(rows), max_pages))
            first = len(rows) - len(members)
            logits, nxt = orc.decoder_step(m, cfg, kp, vp, P, max_pages, tables, tokens, lengths,
                                           logits_from=first)
            print(f"[7b] oracle prompts of requests {list(members)}: {len(rows)} rows", flush=True)
            for j, r in enumerate(members):
                out = outs[r]
                assert_f16_path(out["prefill_logits"], logits[first + j],
                                f"request {r} prefill logits")
                _check_token(int(out["generated_token_ids"][0]), int(nxt[first + j]),
                             logits[first + j], f"request {r} first token")
        step_tables = np.broadcast_to(table, (SHAPE["layers"], batch, max_pages))
        for step in range(steps):
            tok = np.array([out["generated_token_ids"][step] for out in outs], np.int32)
            lens = np.array([len(p) + step + 1 for p in prompts], np.int32)
            logits, nxt = orc.decoder_step(m, cfg, kp, vp, P, max_pages, step_tables, tok, lens)
            for r, out in enumerate(outs):
                assert_f16_path(out["decode_logits"][step], logits[r],
                                f"request {r} decode step {step}")
                _check_token(int(out["generated_token_ids"][step + 1]), int(nxt[r]), logits[r],
                             f"request {r} step {step}")
    finally:
        orc.set_threads(1)


def test_7b_batch1_folded_norms_equal_norm_kernels(host, orc, rt7b, models7b):
    """The one-row bucket with the norms folded into the neighbouring GEMVs
    (o / down + residual epilogue, norm prologue in q.k.v, gate/up and the LM
    head) against the same bucket with the 512-thread norm kernels: logits
    and greedy tokens equal bit for bit over 40 steps that cross pages, with
    2L + 1 fewer dispatches per step."""
    model, plan = models7b(1024)
    runs = {}
    for fold in (True, False):
        pools = [host.create_kv_page_pool(rt7b, plan.kv_plan(), P, 1024 // P)
                 for _ in range(SHAPE["layers"])]
        ex = host.create_batched_decode_executor(rt7b, model, pools, 1, fold_norms=fold)
        states = [host.create_kv_cache_state(rt7b, plan.kv_plan(), pool, False) for pool in pools]
        rng = np.random.default_rng(5101)
        logits, tokens = [], []
        for i in range(40):
            for s in states:
                assert s.stage_length(rt7b, i + 1) == ""
                s.commit_length(i + 1)
            tables = [s.page_table() + [-1] * (ex.max_pages() - len(s.page_table())) for s in states]
            out = ex.run([int(rng.integers(0, SHAPE["vocabulary"]))], [i + 1], tables, True, False)
            assert out["passed"], out["error"]
            logits.append(np.asarray(out["logits"], np.float32))
            tokens.append(int(out["next_token_ids"][0]))
        runs[fold] = (ex.dispatches_per_step(1), logits, tokens)
        del ex, states, pools
    L = SHAPE["layers"]
    assert runs[False][0] - runs[True][0] == 2 * L + 1
    for i, (a, b) in enumerate(zip(runs[True][1], runs[False][1])):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}"
    assert runs[True][2] == runs[False][2]


def test_7b_batch1_attention_output_fusion_matches_two_launches(host, orc, rt7b, models7b):
    """The folded one-row bucket with each layer's paged attention and o
    projection + residual in one launch (fuse_attention_output; the fusion
    candidate of DecoderLLMExecutor.cpp:648-713) against the same bucket with
    the two launches: one dispatch fewer per layer, logits within the fp16
    path tolerance and the same greedy tokens (up to near-ties) over 40 steps
    that cross pages.  The fused kernel sums the o projection per kv head,
    so the two differ by rounding only."""
    model, plan = models7b(1024)
    runs = {}
    for fused in (True, False):
        pools = [host.create_kv_page_pool(rt7b, plan.kv_plan(), P, 1024 // P)
                 for _ in range(SHAPE["layers"])]
        ex = host.create_batched_decode_executor(rt7b, model, pools, 1,
                                                 fuse_attention_output=fused)
        states = [host.create_kv_cache_state(rt7b, plan.kv_plan(), pool, False) for pool in pools]
        rng = np.random.default_rng(5102)
        logits, tokens = [], []
        for i in range(40):
            for s in states:
                assert s.stage_length(rt7b, i + 1) == ""
                s.commit_length(i + 1)
            tables = [s.page_table() + [-1] * (ex.max_pages() - len(s.page_table())) for s in states]
            out = ex.run([int(rng.integers(0, SHAPE["vocabulary"]))], [i + 1], tables, True, False)
            assert out["passed"], out["error"]
            logits.append(np.asarray(out["logits"], np.float32))
            tokens.append(int(out["next_token_ids"][0]))
        runs[fused] = (ex.dispatches_per_step(1), logits, tokens)
        del ex, states, pools
    assert runs[False][0] - runs[True][0] == SHAPE["layers"]
    for i, (a, b) in enumerate(zip(runs[True][1], runs[False][1])):
        assert_f16_path(a, b.astype(np.float64), f"step {i}")
        _check_token(runs[True][2][i], runs[False][2][i], b, f"step {i}")


def test_7b_batch16_folded_norms_match_norm_kernels(host, orc, rt7b, models7b):
    """The 16-row bucket with the norms folded into the packed projections
    (gamma-scaled packed q.k.v, gate/up and LM head weights, 1/rms from the
    residual stream's fragments; o and down + residual) against the same
    bucket with the Add+RMSNorm kernels: logits of every row within the fp16
    path tolerance and the same greedy tokens (up to near-ties) over 24 steps
    that cross a page (every row grows from length 1, so each attended
    position was appended by an earlier step), with 2L fewer dispatches per
    step (the embedding is packed once: one launch more, 2L + 1 norms
    fewer)."""
    model, plan = models7b(1024)
    rows = 16
    runs = {}
    for fold in (True, False):
        # the pool holds one request at full capacity (64 pages), which also
        # covers 16 rows of 2 pages
        pools = [host.create_kv_page_pool(rt7b, plan.kv_plan(), P, 1024 // P)
                 for _ in range(SHAPE["layers"])]
        ex = host.create_batched_decode_executor(rt7b, model, pools, rows, fold_norms=fold)
        mp = ex.max_pages()
        states = [[host.create_kv_cache_state(rt7b, plan.kv_plan(), pool, False) for pool in pools]
                  for _ in range(rows)]
        rng = np.random.default_rng(5103)
        logits, tokens = [], []
        for i in range(24):
            lengths = [i + 1] * rows
            for r in range(rows):
                for s in states[r]:
                    assert s.stage_length(rt7b, lengths[r]) == ""
                    s.commit_length(lengths[r])
            tables = []
            for layer in range(SHAPE["layers"]):
                flat = []
                for r in range(rows):
                    t = states[r][layer].page_table()
                    flat += t + [-1] * (mp - len(t))
                tables.append(flat)
            toks = [int(t) for t in rng.integers(0, SHAPE["vocabulary"], rows)]
            out = ex.run(toks, lengths, tables, True, False)
            assert out["passed"], out["error"]
            logits.append(np.asarray(out["logits"], np.float32).reshape(rows, -1))
            tokens.append([int(t) for t in out["next_token_ids"]])
        runs[fold] = (ex.dispatches_per_step(rows), logits, tokens)
        del ex, states, pools
    assert runs[False][0] - runs[True][0] == 2 * SHAPE["layers"]
    for i, (a, b) in enumerate(zip(runs[True][1], runs[False][1])):
        for r in range(rows):
            assert_f16_path(a[r], b[r].astype(np.float64), f"step {i} row {r}")
            _check_token(runs[True][2][i][r], runs[False][2][i][r], b[r], f"step {i} row {r}")


@pytest.mark.parametrize("batch", [1, 16])
def test_7b_full_depth_chained_steps_equal_serving(host, rt7b, batch):
    """The configuration bench.py times (C5: 32 layers at 7B widths, random
    weights made on the device, prompts ~U[32, 512] through chunked prefill,
    capacity 1024, 16-position pages) checked by properties that hold at any
    depth: the chained decode steps of measureDecodeThroughput (tokens fed
    back on the device, the token-only tail where admitted) generate the
    tokens runContinuousBatch generates for the same requests over 32 decode
    steps, and every logit the serving loop records is finite.  A token may
    differ only where the serving logits' top two are within the fp16-path
    tolerance (2e-2) of each other; the sequences are compared up to there."""
    plan = host.DecoderLLMPlan()
    att = host.KVCachePlan()
    att.heads, att.head_dimension, att.capacity = 32, 128, 1024
    att.dtype = host.DType.Float16
    plan.attention = att
    plan.layer_count, plan.intermediate_size = 32, 11008
    plan.vocabulary_size, plan.rms_norm_epsilon = 32000, 1e-6
    model = host.create_synthetic_model_resources(rt7b, plan, 501)
    rng = np.random.default_rng(502)
    prompts = [list(map(int, rng.integers(0, 32000, rng.integers(32, 513))))
               for _ in range(batch)]
    steps = 32
    print(f"[7b-full] batch {batch}: chained decode", flush=True)
    chained = host.measure_decode_throughput(rt7b, model, prompts, steps, P, False, False, 1024)
    assert chained["passed"], chained["error"]
    specs = []
    for i, prompt in enumerate(prompts):
        spec = host.ServingRequestSpec()
        spec.id = f"r{i}"
        spec.prompt_token_ids = [float(t) for t in prompt]
        spec.decode_token_count = steps
        spec.arrival_step = 0
        specs.append(spec)
    config = host.ServingConfig()
    config.page_size = P
    config.physical_pages_per_layer = max(batch * ((512 + steps + P) // P + 1), 1024 // P)
    config.maximum_batch_size = batch
    config.record_decode_logits = True
    config.prefill_chunk_size = 1024
    config.prefill_requests_per_chunk = batch
    print(f"[7b-full] batch {batch}: serving", flush=True)
    served = host.run_continuous_batch(rt7b, model, specs, config)
    assert served["passed"], served["error"]
    compared, diverged_at_prompt = 0, 0
    for r, out in enumerate(served["requests"]):
        want = [int(t) for t in chained["generated_token_ids"][r]]
        got = [int(t) for t in out["generated_token_ids"]]
        assert len(want) == steps + 1 and len(got) == steps + 1, r
        assert len(out["decode_logits"]) == steps, r
        for s, logits in enumerate(out["decode_logits"]):
            assert np.all(np.isfinite(logits)), f"row {r} step {s}: non-finite logits"
        if got[0] != want[0]:
            # the prompt's last token differs (the two loops pack prompts into
            # chunks on their own): nothing further to compare for this row
            diverged_at_prompt += 1
            continue
        for s in range(1, steps + 1):
            if got[s] != want[s]:
                logits = np.asarray(out["decode_logits"][s - 1])
                gap = abs(float(logits[got[s]]) - float(logits[want[s]]))
                assert gap <= 2e-2, f"row {r} step {s}: token {got[s]} != {want[s]} (gap {gap})"
                break
            compared += 1
    assert diverged_at_prompt <= batch // 8, diverged_at_prompt
    assert compared >= steps * batch * 3 // 4, compared
    if batch > 1:
        assert chained["token_only_available"]
