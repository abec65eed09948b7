"""GPU parity of the decode path through the C++ host layer (HipRuntime ->
C ABI -> gfx950 kernels): CompiledDecoderLLM, the batched decode executor and
the continuous-batching serving loop, against the oracle's decoder step
(oracle/tmc_oracle.c tmco_decoder_step, pinned by test_oracle_decoder.py) on
the same fp16 weights, tokens and block tables.

Tolerances: logits and K/V contents are fp16-path values (2e-2 absolute,
3e-3 relative RMS); greedy tokens must agree unless the oracle's top two
logits are closer than that tolerance.  Page gather/scatter is bit-exact:
a snapshot -> release -> restore round trip into other pages reproduces the
cache bits and the following step's logits bit for bit."""
import numpy as np
import pytest

from tests.helpers import assert_f16_path

pytestmark = pytest.mark.gpu

P = 16  # page size


def _cfg(hidden, heads, head_dim, kv_heads, layers=2, inter=512, vocab=1000, capacity=128):
    return dict(layers=layers, hidden=hidden, heads=heads, head_dim=head_dim, kv_heads=kv_heads,
                intermediate=inter, vocabulary=vocab, capacity=capacity, epsilon=1e-6)


CONFIGS = {
    "mha_d64": _cfg(256, 4, 64, 4),
    "gqa_d128": _cfg(256, 2, 128, 1),
    "gqa4_d128": _cfg(512, 4, 128, 1, layers=1, vocab=3000, capacity=256),
    "serve": _cfg(512, 4, 128, 2, layers=2, vocab=3000, capacity=64),
}


def _weights(orc, cfg, seed):
    rng = np.random.default_rng(seed)
    H, I, V, D = cfg["hidden"], cfg["intermediate"], cfg["vocabulary"], cfg["head_dim"]
    kv = cfg["kv_heads"] * D
    f16 = lambda a: orc.f16(np.asarray(a, np.float32))  # noqa: E731
    w = lambda *shape: f16(rng.standard_normal(shape) * 0.05)  # noqa: E731
    layers = [dict(input_norm=f16(rng.uniform(0.5, 1.5, H)), wq=w(H, H), wk=w(kv, H), wv=w(kv, H),
                   wo=w(H, H), post_norm=f16(rng.uniform(0.5, 1.5, H)), wg=w(I, H), wu=w(I, H),
                   wd=w(H, I)) for _ in range(cfg["layers"])]
    pos = np.arange(cfg["capacity"], dtype=np.float64)[:, None]
    freq = 10000.0 ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    return dict(embedding=f16(rng.standard_normal((V, H))), final_norm=f16(rng.uniform(0.5, 1.5, H)),
                lm_head=w(V, H), rope_cos=np.cos(pos * freq).astype(np.float32),
                rope_sin=np.sin(pos * freq).astype(np.float32), layers=layers)


def _workload(host, orc, cfg, m):
    val = orc.f16_values
    w = host.DecoderLLMWorkload()
    plan = host.DecoderLLMPlan()
    att = host.KVCachePlan()
    att.heads, att.head_dimension, att.capacity = cfg["heads"], cfg["head_dim"], cfg["capacity"]
    att.dtype = host.DType.Float16
    plan.attention = att
    plan.layer_count, plan.intermediate_size = cfg["layers"], cfg["intermediate"]
    plan.vocabulary_size, plan.rms_norm_epsilon = cfg["vocabulary"], cfg["epsilon"]
    plan.key_value_heads = cfg["kv_heads"]
    w.plan = plan
    w.embedding_weight = val(m["embedding"]).ravel()
    w.final_norm_weight = val(m["final_norm"])
    w.language_model_head_weight = val(m["lm_head"]).ravel()
    w.rope_cosine = m["rope_cos"].ravel()
    w.rope_sine = m["rope_sin"].ravel()
    layers = []
    for lw in m["layers"]:
        p = host.DecoderLLMLayerParameters()
        p.input_norm_weight = val(lw["input_norm"])
        p.query_weight = val(lw["wq"]).ravel()
        p.key_weight = val(lw["wk"]).ravel()
        p.value_weight = val(lw["wv"]).ravel()
        p.output_weight = val(lw["wo"]).ravel()
        p.post_attention_norm_weight = val(lw["post_norm"])
        p.gate_weight = val(lw["wg"]).ravel()
        p.up_weight = val(lw["wu"]).ravel()
        p.down_weight = val(lw["wd"]).ravel()
        layers.append(p)
    w.layers = layers
    return w


class OracleRequest:
    """One request replayed on the oracle with its own pools."""

    def __init__(self, orc, cfg, m, pages):
        self.orc, self.cfg, self.m = orc, cfg, m
        self.max_pages = cfg["capacity"] // P
        size = pages * cfg["kv_heads"] * P * cfg["head_dim"]
        self.k = [np.zeros(size, np.uint16) for _ in range(cfg["layers"])]
        self.v = [np.zeros(size, np.uint16) for _ in range(cfg["layers"])]

    def step(self, token, length, tables):
        t = np.full((self.cfg["layers"], 1, self.max_pages), -1, np.int32)
        for l, table in enumerate(tables):
            t[l, 0, :len(table)] = table
        logits, nxt = self.orc.decoder_step(self.m, self.cfg, self.k, self.v, P, self.max_pages, t,
                                            np.array([token]), np.array([length]))
        return logits[0], int(nxt[0])

    def prefix(self, layer, table, length, keys=True):
        kvh, d = self.cfg["kv_heads"], self.cfg["head_dim"]
        pool = (self.k if keys else self.v)[layer].reshape(-1, kvh, P, d)
        out = np.empty((kvh, length, d), np.float32)
        for pos in range(length):
            out[:, pos, :] = self.orc.f16_values(pool[table[pos // P], :, pos % P, :])
        return out


def _check_token(gpu_token, ref_token, ref_logits, what):
    if gpu_token != ref_token:
        top = np.sort(ref_logits)[-2:]
        assert top[1] - top[0] <= 2e-2, f"{what}: token {gpu_token} != {ref_token}"


@pytest.fixture(scope="module")
def rt(host):
    r = host.HipRuntime()
    assert r.is_available(), r.initialization_error()
    return r


@pytest.mark.parametrize("name", list(CONFIGS))
def test_compiled_decoder_matches_oracle(host, orc, rt, name):
    cfg = CONFIGS[name]
    m = _weights(orc, cfg, 11)
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    dec, log = host.compile_decoder_llm(rt, _workload(host, orc, cfg, m), opts)
    assert "dispatches/token" in log
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, cfg["vocabulary"], 21)
    res = dec.prefill([float(t) for t in prompt], True)
    assert res["passed"], res["error"]
    V = cfg["vocabulary"]
    gpu_logits = res["logits"].reshape(len(prompt), V)
    tables = [dec.kv_block_table(l) for l in range(cfg["layers"])]
    ref = OracleRequest(orc, cfg, m, cfg["capacity"] // P)
    for i, tok in enumerate(prompt):
        logits, nxt = ref.step(int(tok), i + 1, tables)
        assert_f16_path(gpu_logits[i], logits, f"{name} prefill position {i}")
    _check_token(int(res["next_token_ids"][0]), nxt, logits, f"{name} first token")
    token = int(res["next_token_ids"][0])
    for step in range(6):
        out = dec.decode([float(token)], True)
        assert out["passed"], out["error"]
        length = len(prompt) + step + 1
        tables = [dec.kv_block_table(l) for l in range(cfg["layers"])]
        logits, nxt = ref.step(token, length, tables)
        assert_f16_path(out["logits"], logits, f"{name} decode step {step}")
        _check_token(int(out["next_token_ids"][0]), nxt, logits, f"{name} step {step}")
        token = int(out["next_token_ids"][0])
    length = dec.current_length()
    assert length == len(prompt) + 6
    kvh, d = cfg["kv_heads"], cfg["head_dim"]
    for l in range(cfg["layers"]):
        table = dec.kv_block_table(l)
        assert_f16_path(dec.read_key_prefix(l).reshape(kvh, length, d),
                        ref.prefix(l, table, length, True), f"{name} layer {l} keys")
        assert_f16_path(dec.read_value_prefix(l).reshape(kvh, length, d),
                        ref.prefix(l, table, length, False), f"{name} layer {l} values")


def test_decoder_rules_and_contiguous_cache(host, orc, rt):
    cfg = CONFIGS["mha_d64"]
    m = _weights(orc, cfg, 21)
    w = _workload(host, orc, cfg, m)
    paged_opts = host.DecoderLLMCompileOptions()
    paged_opts.kv_page_size = P
    paged, _ = host.compile_decoder_llm(rt, w, paged_opts)
    flat, _ = host.compile_decoder_llm(rt, w, host.DecoderLLMCompileOptions())
    assert flat.uses_paged_kv_cache() is False and paged.uses_paged_kv_cache() is True
    out = paged.decode([1.0], True)
    assert not out["passed"] and "prefill" in out["error"]
    prompt = [float(t) for t in np.random.default_rng(3).integers(0, cfg["vocabulary"], 9)]
    a = paged.prefill(prompt, True)
    b = flat.prefill(prompt, True)
    assert a["passed"] and b["passed"]
    # One page of `capacity` tokens and 16-token pages run the same kernels on
    # the same positions: the logits agree bit for bit.
    np.testing.assert_array_equal(a["logits"], b["logits"])
    assert not paged.prefill(prompt, True)["passed"]  # cache not empty
    bad = paged.decode([float(cfg["vocabulary"])], True)
    assert not bad["passed"] and "vocabulary" in bad["error"]
    assert paged.current_length() == len(prompt)  # rolled back
    assert paged.reset() == "" and paged.current_length() == 0


def test_decoder_capacity_reached_leaves_state_unchanged(host, orc, rt):
    """DecoderLLMExecutor.cpp:1043-1046: at capacity the decoder refuses the
    step with "Decoder KV cache capacity has been reached." and keeps its
    length, pages and cache bits; a prompt beyond the capacity is refused
    before any page is taken."""
    cfg = dict(CONFIGS["gqa_d128"], capacity=32)
    m = _weights(orc, cfg, 91)
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    dec, _ = host.compile_decoder_llm(rt, _workload(host, orc, cfg, m), opts)
    too_long = dec.prefill([1.0] * 33, False)
    assert not too_long["passed"] and dec.current_length() == 0
    assert dec.allocated_kv_page_count() == 0
    assert dec.prefill([float(t) for t in range(3, 33)], False)["passed"]
    token = 7.0
    for _ in range(2):
        out = dec.decode([token], True)
        assert out["passed"], out["error"]
        token = float(out["next_token_ids"][0])
    assert dec.current_length() == 32 and dec.allocated_kv_page_count() == 2
    keys = [dec.read_key_prefix(l) for l in range(cfg["layers"])]
    values = [dec.read_value_prefix(l) for l in range(cfg["layers"])]
    tables = [dec.kv_block_table(l) for l in range(cfg["layers"])]
    full = dec.decode([token], True)
    assert not full["passed"] and full["error"] == "Decoder KV cache capacity has been reached."
    assert dec.current_length() == 32 and dec.allocated_kv_page_count() == 2
    assert [dec.kv_block_table(l) for l in range(cfg["layers"])] == tables
    for l in range(cfg["layers"]):
        assert np.array_equal(dec.read_key_prefix(l), keys[l])
        assert np.array_equal(dec.read_value_prefix(l), values[l])


def test_snapshot_restore_moves_pages_bit_exactly(host, orc, rt):
    cfg = CONFIGS["gqa_d128"]
    m = _weights(orc, cfg, 31)
    w = _workload(host, orc, cfg, m)
    pools = [host.create_kv_page_pool(rt, w.plan.kv_plan(), P, 32) for _ in range(cfg["layers"])]
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    opts.shared_kv_pools = pools
    a, _ = host.compile_decoder_llm(rt, w, opts)
    opts.shared_model_resources = a.shared_model_resources()
    b, _ = host.compile_decoder_llm(rt, w, opts)
    prompt = [float(t) for t in np.random.default_rng(4).integers(0, cfg["vocabulary"], 37)]
    assert b.prefill(prompt, False)["passed"]
    before = [b.kv_block_table(l) for l in range(cfg["layers"])]
    keys = [b.read_key_prefix(l) for l in range(cfg["layers"])]
    snap = b.snapshot_kv_cache()
    assert b.release_kv_cache() == "" and b.current_length() == 0
    assert a.prefill(prompt[:20], False)["passed"]  # takes b's old pages
    assert b.restore_kv_cache(snap) == ""
    after = [b.kv_block_table(l) for l in range(cfg["layers"])]
    assert after != before
    for l in range(cfg["layers"]):
        np.testing.assert_array_equal(b.read_key_prefix(l), keys[l])
    # Same cache contents in other pages: the next step is bit-identical to a
    # fresh request that never moved.
    c_opts = host.DecoderLLMCompileOptions()
    c_opts.kv_page_size = P
    c_opts.shared_model_resources = a.shared_model_resources()
    c, _ = host.compile_decoder_llm(rt, w, c_opts)
    assert c.prefill(prompt, False)["passed"]
    x = b.decode([5.0], True)
    y = c.decode([5.0], True)
    assert x["passed"] and y["passed"]
    np.testing.assert_array_equal(x["logits"], y["logits"])


def test_failed_step_rolls_back(host, orc, rt):
    cfg = CONFIGS["mha_d64"]
    m = _weights(orc, cfg, 41)
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    w = _workload(host, orc, cfg, m)
    dec, _ = host.compile_decoder_llm(rt, w, opts)
    prompt = [float(t) for t in range(1, 17)]  # fills exactly one page
    assert dec.prefill(prompt, False)["passed"]
    want = dec.decode([7.0], True)  # needs a second page
    assert want["passed"] and dec.allocated_kv_page_count() == 2
    opts.shared_model_resources = dec.shared_model_resources()
    dec2, _ = host.compile_decoder_llm(rt, w, opts)
    assert dec2.prefill(prompt, False)["passed"]
    assert dec2.allocated_kv_page_count() == 1
    rt.fail_next(1)
    out = dec2.decode([7.0], True)
    assert not out["passed"] and "Injected" in out["error"]
    # the staged page was released and the length kept
    assert dec2.current_length() == 16 and dec2.allocated_kv_page_count() == 1
    again = dec2.decode([7.0], True)
    assert again["passed"]
    np.testing.assert_array_equal(again["logits"], want["logits"])


def test_batched_executor_rows_match_oracle(host, orc, rt):
    cfg = CONFIGS["gqa4_d128"]
    m = _weights(orc, cfg, 51)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    pages = 48
    pools = [host.create_kv_page_pool(rt, w.plan.kv_plan(), P, pages) for _ in range(cfg["layers"])]
    ex = host.create_batched_decode_executor(rt, model, pools, 5)
    assert ex.buckets() == [1, 2, 4, 5]
    max_pages = ex.max_pages()
    rng = np.random.default_rng(52)
    lengths = [1, 17, 40, 3, 16]
    # each row gets its own pages, allocated through KV states over the pools
    states = [[host.create_kv_cache_state(rt, w.plan.kv_plan(), pools[l], False)
               for l in range(cfg["layers"])] for _ in lengths]
    refs = [OracleRequest(orc, cfg, m, pages) for _ in lengths]
    history = [rng.integers(0, cfg["vocabulary"], n) for n in lengths]
    # fill every row's history one token at a time through one-row steps
    for r, hist in enumerate(history):
        for i, tok in enumerate(hist[:-1]):
            for s in states[r]:
                assert s.stage_length(rt, i + 1) == ""
                s.commit_length(i + 1)
            tables = [s.page_table() + [-1] * (max_pages - len(s.page_table())) for s in states[r]]
            out = ex.run([int(tok)], [i + 1], tables, False, False)
            assert out["passed"], out["error"]
            refs[r].step(int(tok), i + 1, [s.page_table() for s in states[r]])
    # one batched step over all rows (their last history token)
    for r, n in enumerate(lengths):
        for s in states[r]:
            assert s.stage_length(rt, n) == ""
    tables = [[] for _ in range(cfg["layers"])]
    for r in range(len(lengths)):
        for l, s in enumerate(states[r]):
            tables[l] += s.page_table() + [-1] * (max_pages - len(s.page_table()))
    out = ex.run([int(h[-1]) for h in history], lengths, tables, True, True)
    assert out["passed"], out["error"]
    assert out["gpu_us"] is not None and out["gpu_us"] > 0
    V = cfg["vocabulary"]
    for r, n in enumerate(lengths):
        logits, nxt = refs[r].step(int(history[r][-1]), n, [s.page_table() for s in states[r]])
        assert_f16_path(out["logits"][r * V:(r + 1) * V], logits, f"row {r}")
        _check_token(int(out["next_token_ids"][r]), nxt, logits, f"row {r}")
    # host checks: unallocated page, token outside the vocabulary, bad length
    bad = [list(t) for t in tables]
    bad[0][0] = [p for p in range(pages) if p not in tables[0]][0]
    assert "not allocated" in ex.run([1] * 5, lengths, bad, False, False)["error"]
    assert "vocabulary" in ex.run([V] + [1] * 4, lengths, tables, False, False)["error"]
    assert "capacity" in ex.run([1] * 5, [0] + lengths[1:], tables, False, False)["error"]


def test_launch_chained_matches_run_with_a_repeated_length(host, orc, rt):
    """BatchedDecodeExecutor.launch_chained against run(): three rows decode
    from empty caches across page boundaries.  The chained executor keeps each
    step's greedy tokens and the lengths advanced by one on the device (one
    tmc_decode_chain launch between steps); one step repeats the previous
    length (a rollback by one position), so its lengths do not follow and go
    up again.  Every step's tokens equal those of a second executor over its
    own pools that reads each step's tokens back and uploads them (run)."""
    cfg = CONFIGS["serve"]
    m = _weights(orc, cfg, 81)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    L, rows, pages = cfg["layers"], 3, 16
    execs, states = [], []
    for _ in range(2):
        pools = [host.create_kv_page_pool(rt, w.plan.kv_plan(), P, pages) for _ in range(L)]
        execs.append(host.create_batched_decode_executor(rt, model, pools, rows))
        states.append([[host.create_kv_cache_state(rt, w.plan.kv_plan(), pools[l], False)
                        for l in range(L)] for _ in range(rows)])
    max_pages = execs[0].max_pages()
    schedule = list(range(1, 21)) + [20] + list(range(21, 41))

    def stage(e, n):
        tables = [[] for _ in range(L)]
        for r in range(rows):
            for l, st in enumerate(states[e][r]):
                assert st.stage_length(rt, n) == ""
                st.commit_length(n)
                tables[l] += st.page_table() + [-1] * (max_pages - len(st.page_table()))
        return tables

    first = [11, 222, 2999]
    chained, stepped = execs
    chained.reserve_history(len(schedule))
    want, tokens = [], list(first)
    for step, n in enumerate(schedule):
        chained.launch_chained(first if step == 0 else [], [n] * rows, stage(0, n), step)
        out = stepped.run(tokens, [n] * rows, stage(1, n), False, False)
        assert out["passed"], out["error"]
        tokens = [int(t) for t in out["next_token_ids"]]
        want.append(tokens)
    got = chained.read_history(len(schedule))
    for step in range(len(schedule)):
        assert list(got[step * rows:(step + 1) * rows]) == want[step], step
    # a chained step without tokens needs the previous step's row count
    with pytest.raises(RuntimeError, match="row count"):
        chained.launch_chained([], [41, 41], stage(0, 41), 0)


@pytest.mark.parametrize("chunk,per_chunk", [(0, 1), (8, 1), (64, 4)])
def test_serving_matches_single_request_decoding(host, orc, rt, chunk, per_chunk):
    """chunk 0: prompts by decode in the batched ticks; chunk > 0: prompts
    in chunks through the chunked prefill executor at admission, one request
    per chunk or up to four packed together."""
    cfg = CONFIGS["serve"]
    m = _weights(orc, cfg, 61)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    rng = np.random.default_rng(62)
    specs = []
    for i in range(5):
        s = host.ServingRequestSpec()
        s.id = f"q{i}"
        s.prompt_token_ids = [float(t) for t in rng.integers(0, cfg["vocabulary"], rng.integers(5, 30))]
        s.decode_token_count = int(rng.integers(1, 12))
        s.arrival_step = int(rng.integers(0, 6))
        specs.append(s)
    config = host.ServingConfig()
    config.page_size = P
    config.physical_pages_per_layer = 6  # 4 pages hold one full request: page pressure
    config.record_decode_logits = True
    config.prefill_chunk_size = chunk
    config.prefill_requests_per_chunk = per_chunk
    result = host.run_continuous_batch(rt, model, specs, config)
    assert result["passed"], result["error"]
    metrics = result["metrics"]
    assert (metrics["prefill_chunk_submissions"] > 0) == (chunk > 0)
    assert metrics["decoded_tokens"] == sum(s.decode_token_count for s in specs)
    assert metrics["maximum_active_batch_size"] > 1
    # page pressure preempts: the KV pages spill raw to pinned host memory
    # (prompts consumed at admission change the schedule: no preemption is
    # required there)
    if chunk == 0:
        assert metrics["preemption_count"] > 0 and metrics["spilled_bytes"] > 0
    assert (metrics["spilled_bytes"] > 0) == (metrics["preemption_count"] > 0)
    assert metrics["resume_count"] == metrics["preemption_count"]
    print("serving metrics:", {k: v for k, v in metrics.items() if not isinstance(v, dict)})
    # oracle replay of every request: its prompt as one step (rows in
    # position order), then one step per generated token, on the oracle's
    # own pools; the serving loop's logits must match at every step
    V = cfg["vocabulary"]
    for spec, out in zip(specs, result["requests"]):
        ref = OracleRequest(orc, cfg, m, cfg["capacity"] // P)
        prompt = np.asarray(spec.prompt_token_ids, np.int32)
        n = len(prompt)
        table = np.arange(cfg["capacity"] // P, dtype=np.int32)
        t = np.broadcast_to(table, (cfg["layers"], n, table.size))
        logits, nxt = orc.decoder_step(m, cfg, ref.k, ref.v, P, table.size, t, prompt,
                                       np.arange(1, n + 1), logits_from=n - 1)
        assert_f16_path(out["prefill_logits"], logits[-1], f"{spec.id} prefill vs oracle")
        gen = out["generated_token_ids"]
        _check_token(int(gen[0]), int(nxt[-1]), logits[-1], f"{spec.id} first token vs oracle")
        for i in range(spec.decode_token_count):
            lg, nx = ref.step(int(gen[i]), n + i + 1, [table] * cfg["layers"])
            assert_f16_path(out["decode_logits"][i], lg, f"{spec.id} step {i} vs oracle")
            _check_token(int(gen[i + 1]), nx, lg, f"{spec.id} step {i} token vs oracle")
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    opts.shared_model_resources = model
    for spec, out in zip(specs, result["requests"]):
        dec, _ = host.compile_decoder_llm(rt, w, opts)
        first = dec.prefill(spec.prompt_token_ids, True)
        V = cfg["vocabulary"]
        assert_f16_path(out["prefill_logits"], first["logits"][-V:], f"{spec.id} prefill")
        gen = out["generated_token_ids"]
        assert len(gen) == spec.decode_token_count + 1
        _check_token(int(gen[0]), int(first["next_token_ids"][0]), first["logits"][-V:], spec.id)
        if int(gen[0]) != int(first["next_token_ids"][0]):
            continue  # near-tie: the sequences legitimately diverge here
        for i in range(spec.decode_token_count):
            step = dec.decode([gen[i]], True)
            assert_f16_path(out["decode_logits"][i], step["logits"], f"{spec.id} step {i}")
            if int(step["next_token_ids"][0]) != int(gen[i + 1]):
                _check_token(int(gen[i + 1]), int(step["next_token_ids"][0]), step["logits"],
                             f"{spec.id} step {i}")
                break


@pytest.mark.parametrize("chunk", [0, 16])
def test_chained_decode_throughput_matches_stepped(host, orc, rt, chunk):
    """measureDecodeThroughput's chained steps (greedy tokens fed back on the
    device, read once at the end) generate exactly the tokens of the stepped
    loop (one host round trip per step, the timeGpu path), batch 3 with
    ragged prompts crossing page boundaries; and the first generated token
    of each row equals the one-request decoder's."""
    cfg = CONFIGS["serve"]
    m = _weights(orc, cfg, 71)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    rng = np.random.default_rng(72)
    prompts = [list(map(int, rng.integers(0, cfg["vocabulary"], n))) for n in (5, 17, 30)]
    decode = 20
    chained = host.measure_decode_throughput(rt, model, prompts, decode, P, False, False, chunk)
    stepped = host.measure_decode_throughput(rt, model, prompts, decode, P, True, False, chunk)
    assert chained["passed"], chained["error"]
    assert stepped["passed"], stepped["error"]
    assert stepped["step_gpu"]["samples"] == decode
    for r, (a, b) in enumerate(zip(chained["generated_token_ids"], stepped["generated_token_ids"])):
        assert len(a) == decode + 1, r
        assert [int(t) for t in a] == [int(t) for t in b], r
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    opts.shared_model_resources = model
    for r, prompt in enumerate(prompts):
        dec, _ = host.compile_decoder_llm(rt, w, opts)
        first = dec.prefill([float(t) for t in prompt], True)
        V = cfg["vocabulary"]
        _check_token(int(chained["generated_token_ids"][r][0]), int(first["next_token_ids"][0]),
                     first["logits"][-V:], f"row {r}")


def test_tuned_executor_matches_default_and_caches_shapes(host, orc, rt):
    """Batch-1 GEMVs with the decode GEMV tuner's per-shape selections: the
    shapes are tuned once (process cache), and the step's logits match the
    default-configuration executor within the fp16-path tolerance."""
    cfg = CONFIGS["gqa4_d128"]
    m = _weights(orc, cfg, 61)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    host.clear_decode_gemv_cache()
    runs = []
    for tune in (False, True, True):
        pools = [host.create_kv_page_pool(rt, w.plan.kv_plan(), P, 16)
                 for _ in range(cfg["layers"])]
        ex = host.create_batched_decode_executor(rt, model, pools, 1, tune_kernels=tune)
        states = [host.create_kv_cache_state(rt, w.plan.kv_plan(), pools[l], False)
                  for l in range(cfg["layers"])]
        logits = None
        for i, tok in enumerate([3, 14, 15, 92, 65]):
            for s in states:
                assert s.stage_length(rt, i + 1) == ""
                s.commit_length(i + 1)
            tables = [s.page_table() + [-1] * (ex.max_pages() - len(s.page_table())) for s in states]
            out = ex.run([tok], [i + 1], tables, True, False)
            assert out["passed"], out["error"]
            logits = np.asarray(out["logits"])
        runs.append(logits)
        # q.k.v, o, down and the LM head shapes (distinct ones) are cached
        # after the first tuned build
        H, I, V = cfg["hidden"], cfg["intermediate"], cfg["vocabulary"]
        qkv = H + 2 * cfg["kv_heads"] * cfg["head_dim"]
        shapes = {(H, qkv, "f16"), (H, H, "f16"), (I, H, "f16"), (H, V, "f32")}
        assert host.decode_gemv_cache_size() == (0 if not tune else len(shapes))
    assert_f16_path(runs[1], runs[0], "tuned vs default")
    np.testing.assert_array_equal(runs[2], runs[1])  # the cached selection is the same


def test_token_only_tail_matches_logits_tail(host, orc, rt):
    """The token-only tail (LM head partial argmax + final argmax,
    DecoderLLMExecutor.cpp:837-845) gives the logits tail's tokens step for
    step: two executors over the same weights and histories, one forced to
    the logits tail ("never"), one to the token tail ("always"), steps of 1,
    3 and 5 rows (the one-row bucket folds the norms into the dot GEMV, the
    others run the packed GEMM) with no logits read; every token also agrees
    with the oracle's decoder step.  A third executor under the admission
    rule times both tails on its first logits-free step and records the
    decision and the speedup (two paired rounds)."""
    cfg = CONFIGS["serve"]
    m = _weights(orc, cfg, 91)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    pages, L, V = 64, cfg["layers"], cfg["vocabulary"]
    execs, all_states = [], []
    for policy in ("never", "always"):
        pools = [host.create_kv_page_pool(rt, w.plan.kv_plan(), P, pages) for _ in range(L)]
        ex = host.create_batched_decode_executor(rt, model, pools, 5)
        ex.set_token_only_policy(policy)
        execs.append(ex)
        all_states.append([[host.create_kv_cache_state(rt, w.plan.kv_plan(), pools[l], False)
                            for l in range(L)] for _ in range(5)])
    refs = [OracleRequest(orc, cfg, m, pages) for _ in range(5)]
    rng = np.random.default_rng(92)
    tokens = [int(t) for t in rng.integers(0, V, 5)]
    lengths = [0] * 5
    for rows in (1, 3, 5, 5, 1, 3):
        got = []
        for ex, states in zip(execs, all_states):
            tables = [[] for _ in range(L)]
            for r in range(rows):
                for l, s in enumerate(states[r]):
                    assert s.stage_length(rt, lengths[r] + 1) == ""
                    tables[l] += s.page_table() + [-1] * (ex.max_pages() - len(s.page_table()))
            out = ex.run(tokens[:rows], [n + 1 for n in lengths[:rows]], tables, False, False)
            assert out["passed"], out["error"]
            assert len(out["logits"]) == 0
            for r in range(rows):
                for s in states[r]:
                    s.commit_length(lengths[r] + 1)
            got.append([int(t) for t in out["next_token_ids"]])
        assert got[0] == got[1], rows
        for r in range(rows):
            logits, nxt = refs[r].step(tokens[r], lengths[r] + 1,
                                       [s.page_table() for s in all_states[0][r]])
            _check_token(got[1][r], nxt, logits, f"{rows} rows, row {r}")
            lengths[r] += 1
            tokens[r] = got[1][r]
    for rows in (1, 3, 5):
        st = execs[1].token_only_status(rows)
        assert st["available"] and st["checked"] and st["admitted"], (rows, st)
        assert not execs[0].token_only_status(rows)["admitted"]
    # the admission rule: both tails timed on the first logits-free step
    pools = [host.create_kv_page_pool(rt, w.plan.kv_plan(), P, pages) for _ in range(L)]
    ex = host.create_batched_decode_executor(rt, model, pools, 2)
    states = [host.create_kv_cache_state(rt, w.plan.kv_plan(), pools[l], False) for l in range(L)]
    for s in states:
        assert s.stage_length(rt, 1) == ""
    tables = [s.page_table() + [-1] * (ex.max_pages() - len(s.page_table())) for s in states]
    ex.admit_token_only([7], [1], tables)
    st = ex.token_only_status(1)
    assert st["checked"] and st["speedup"] > 0.0
    assert st["admitted"] == (st["speedup"] >= 1.05)
    out = ex.run([7], [1], tables, False, False)
    assert out["passed"], out["error"]
    logits, nxt = OracleRequest(orc, cfg, m, pages).step(7, 1, [s.page_table() for s in states])
    _check_token(int(out["next_token_ids"][0]), nxt, logits, "admission executor")
