"""GPU parity of the chunked prefill path (prefillChunked,
DecoderLLMExecutor.cpp:982-1034): the prompt GEMM (emitTiledGEMM,
DecodeGEMVMetalEmitter.cpp:134-169), the shared-table RoPE + cache append,
causal chunk attention (emitPagedKVAttention with causalPrefill,
KVCacheMetalEmitter.cpp:159-163,210-310) and the chunked executor, against
the oracle (linear, causal_prefill_attention, decoder_step over the chunk's
rows).

Tolerances as everywhere: fp32 outputs within 1e-4 relative, fp16-path
values within 2e-2 absolute and 3e-3 relative RMS; the RoPE + append is
bit-exact against the per-row decode form."""
import numpy as np
import pytest

from tests.helpers import F16, F32, assert_f16_path, assert_f32_rel, bits, dev, dev_f16, normal, values
from tests.test_decoder_gpu import CONFIGS, OracleRequest, P, _check_token, _weights, _workload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    if not t.cuda.is_available():
        pytest.skip("no GPU")
    return t


@pytest.fixture(scope="module")
def rt(host):
    r = host.HipRuntime()
    assert r.is_available(), r.initialization_error()
    return r


# ---------------------------------------------------------------- prompt GEMM
@pytest.mark.parametrize("m,k,n,out,ws", [(1, 64, 48, F16, False), (37, 256, 200, F16, True),
                                          (64, 512, 1000, F32, True), (300, 1024, 768, F16, False),
                                          (512, 4096, 4096, F16, True),
                                          # split K over the workspace (few output tiles)
                                          (37, 4096, 200, F16, True), (130, 4104, 4100, F32, True),
                                          # ragged m, n and k (k % 64 != 0) without a split
                                          (130, 4104, 4100, F16, False)])
def test_gemm_rows_matches_oracle(tmc, orc, torch, m, k, n, out, ws):
    """The MFMA prompt GEMM (emitTiledGEMM semantics) against the oracle, with
    and without the split-K workspace; repeated calls are bit-identical."""
    x = orc.f16(normal(700 + m, (m, k)))
    w = orc.f16(normal(701 + n, (n, k), 0.03))
    dtype = torch.float16 if out == F16 else torch.float32
    workspace = (torch.empty(tmc.gemm_rows_workspace_bytes() // 4, dtype=torch.int32, device="cuda")
                 if ws else None)
    xd, wd = dev_f16(x), dev_f16(w)
    y = torch.full((m, n), float("nan"), dtype=dtype, device="cuda")
    tmc.gemm_rows(xd, wd, y, workspace)
    y2 = torch.full_like(y, float("nan"))
    tmc.gemm_rows(xd, wd, y2, workspace)
    y3 = torch.full_like(y, float("nan"))
    tmc.gemm_rows(xd, wd, y3, workspace)
    torch.cuda.synchronize()
    ref = orc.linear(x, w, F16)  # exact sums of the fp16 inputs
    what = f"gemm_rows m={m} k={k} n={n}"
    if out == F16:
        assert_f16_path(values(y), ref, what=what)
    else:
        assert_f32_rel(values(y), ref, what=what)
    # deterministic: the split partials are added in split order
    assert torch.equal(y, y2) and torch.equal(y2, y3)
    # the no-workspace entry (never splits) agrees within the same tolerance
    y4 = torch.full_like(y, float("nan"))
    tmc.gemm_mfma(xd, wd, y4)
    torch.cuda.synchronize()
    if out == F16:
        assert_f16_path(values(y4), ref, what=what + " (no split)")
    else:
        assert_f32_rel(values(y4), ref, what=what + " (no split)")


def test_gemm_rows_rejects_bad_arguments(tmc, torch):
    x = torch.zeros((4, 64), dtype=torch.float16, device="cuda")
    w = torch.zeros((8, 64), dtype=torch.float16, device="cuda")
    y = torch.zeros((4, 8), dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="f16 or f32"):
        tmc.gemm_rows(x, w, y)


# --------------------------------------------------------- RoPE + cache append
@pytest.mark.parametrize("qh,kvh,d", [(4, 4, 64), (8, 2, 128)])
def test_prefill_rope_append_equals_decode_form(tmc, orc, torch, qh, kvh, d):
    """Every row shares one table: the result is bit-identical to the decode
    form with the table repeated per row."""
    cap, p, rows, start = 128, 16, 37, 20
    max_pages = cap // p
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos, sin = np.cos(pos * freq).astype(np.float32), np.sin(pos * freq).astype(np.float32)
    qkv = orc.f16(normal(720, (rows, (qh + 2 * kvh) * d)))
    pages = 12
    table = np.random.default_rng(721).permutation(pages)[:max_pages].astype(np.int32)
    lengths = (start + np.arange(rows) + 1).astype(np.int32)
    active = rows - 3  # the last three rows are padding
    pool0 = orc.f16(normal(722, (pages, kvh, p, d)))
    act = torch.tensor([active], dtype=torch.int32, device="cuda")
    outs = []
    for shared in (True, False):
        kp, vp = dev_f16(pool0), dev_f16(pool0.copy())
        q_out = torch.full((rows, qh * d), float("nan"), dtype=torch.float16, device="cuda")
        if shared:
            tmc.prefill_rope_append(dev_f16(qkv), dev(cos), dev(sin), dev(lengths), dev(table), act,
                                    q_out, kp, vp, rows, qh, kvh, d, cap, p, max_pages)
        else:
            tables = np.tile(table, (rows, 1))
            tmc.decode_rope_append(dev_f16(qkv), dev(cos), dev(sin), dev(lengths), dev(tables), act,
                                   q_out, kp, vp, rows, qh, kvh, d, cap, p, max_pages)
        torch.cuda.synchronize()
        outs.append((bits(q_out), bits(kp), bits(vp)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    # padding rows keep their query output
    assert np.all(outs[0][0][active:] == 0x7e00)


# ------------------------------------------------------------ causal attention
CASES = [
    # rows, q_heads, kv_heads, head_dim, page_size, start, active
    (1, 4, 4, 64, 16, 0, None),
    (37, 4, 1, 128, 16, 5, None),
    (64, 8, 8, 128, 16, 100, None),
    (100, 16, 2, 128, 12, 33, 90),
    (130, 32, 8, 128, 16, 200, None),
    (48, 16, 1, 64, 5, 7, None),
    (256, 8, 8, 128, 16, 1000, None),
    (16, 4, 2, 128, 1, 7990, None),  # 8007-entry table: read from global memory, not LDS
]


@pytest.mark.parametrize("rows,qh,kvh,d,p,start,active", CASES)
def test_prefill_attention_matches_oracle(tmc, orc, torch, rows, qh, kvh, d, p, start, active):
    valid = start + rows
    max_pages = (valid + p - 1) // p + 1
    pages = max_pages + 3
    rng = np.random.default_rng(730 + rows)
    table = rng.permutation(pages)[:max_pages].astype(np.int32)
    k_pool = orc.f16(normal(731, (pages, kvh, p, d)))
    v_pool = orc.f16(normal(732, (pages, kvh, p, d)))
    q = orc.f16(normal(733, (rows, qh * d)))
    act = rows if active is None else active
    lengths = (start + np.arange(rows) + 1).astype(np.int32)
    out = torch.full((rows, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.prefill_attention(dev_f16(q), dev_f16(k_pool), dev_f16(v_pool), dev(lengths), dev(table),
                          torch.tensor([act], dtype=torch.int32, device="cuda"), out, rows, qh, kvh,
                          d, p, max_pages, kvh * p * d, p * d)
    torch.cuda.synchronize()
    ref, written = orc.causal_prefill_attention(q, k_pool, v_pool, F16, qh, kvh, d, p, kvh * p * d,
                                                p * d, table, max_pages, valid, rows, act)
    got = values(out)
    assert written[:act].all() and not written[act:].any()
    assert_f16_path(got[:act], ref[:act], what=f"prefill attention rows={rows} qh={qh} kvh={kvh}")
    assert np.isnan(got[act:]).all()


def test_prefill_attention_absent_page_leaves_rows_untouched(tmc, orc, torch):
    """Rows whose causal range reaches an absent page entry (negative, or past
    the pool) keep their output; rows below it are computed."""
    rows, qh, kvh, d, p, start = 40, 4, 2, 128, 16, 8
    max_pages = 4
    pages = 10
    k_pool = orc.f16(normal(740, (pages, kvh, p, d)))
    v_pool = orc.f16(normal(741, (pages, kvh, p, d)))
    q = orc.f16(normal(742, (rows, qh * d)))
    lengths = (start + np.arange(rows) + 1).astype(np.int32)
    for bad in (-1, pages + 5):
        table = np.array([3, 7, bad, 1], np.int32)  # positions 32.. have no page
        out = torch.full((rows, qh * d), float("nan"), dtype=torch.float16, device="cuda")
        tmc.prefill_attention(dev_f16(q), dev_f16(k_pool), dev_f16(v_pool), dev(lengths),
                              dev(table), torch.tensor([rows], dtype=torch.int32, device="cuda"),
                              out, rows, qh, kvh, d, p, max_pages, kvh * p * d, p * d)
        torch.cuda.synchronize()
        got = values(out)
        ok = lengths <= 2 * p
        oracle_table = table.copy()
        oracle_table[2] = -1
        ref, written = orc.causal_prefill_attention(q, k_pool, v_pool, F16, qh, kvh, d, p,
                                                    kvh * p * d, p * d, oracle_table, max_pages,
                                                    start + rows, rows)
        assert list(written.all(axis=1)) == list(ok)
        assert np.isnan(got[~ok]).all()
        assert_f16_path(got[ok], ref[ok], what=f"rows before the absent page ({bad})")


def test_prefill_attention_rejects_bad_shapes(tmc, torch):
    z = torch.zeros(64 * 3 * 128, dtype=torch.float16, device="cuda")
    i = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="head_dim"):
        tmc.prefill_attention(z, z, z, i, i, i, z, 4, 2, 2, 96, 16, 4, 2 * 16 * 96, 16 * 96)
    with pytest.raises(RuntimeError, match="divide 64"):
        tmc.prefill_attention(z, z, z, i, i, i, z, 4, 3, 1, 64, 16, 4, 16 * 64, 16 * 64)


# ------------------------------------------------------------- the executor
def _oracle_chunks(orc, cfg, m, ref, tables, prompt, chunk):
    """Run the prompt through the oracle's decoder step, one step per chunk
    with the chunk's tokens as rows (lengths start + r + 1, the request's
    tables on every row): the causal chunk semantics."""
    L, max_pages, V = cfg["layers"], ref.max_pages, cfg["vocabulary"]
    logits = []
    nxt = None
    for s in range(0, len(prompt), chunk):
        toks = np.asarray(prompt[s:s + chunk])
        t = np.full((L, len(toks), max_pages), -1, np.int32)
        for l, table in enumerate(tables):
            t[l, :, :len(table)] = table
        lg, nxt = orc.decoder_step(m, cfg, ref.k, ref.v, P, max_pages, t, toks,
                                   s + np.arange(len(toks)) + 1)
        logits.append(lg)
    return np.concatenate(logits).reshape(-1, V), nxt


@pytest.mark.parametrize("name,chunk,length", [("mha_d64", 16, 37), ("gqa_d128", 8, 21),
                                               ("gqa4_d128", 64, 130), ("serve", 16, 16)])
def test_prefill_chunked_matches_oracle(host, orc, rt, name, chunk, length):
    cfg = CONFIGS[name]
    m = _weights(orc, cfg, 11)
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    opts.prefill_chunk_size = chunk
    dec, log = host.compile_decoder_llm(rt, _workload(host, orc, cfg, m), opts)
    assert "Chunked prefill stage" in log and dec.prefill_chunk_size() == chunk
    prompt = np.random.default_rng(13).integers(0, cfg["vocabulary"], length)
    res = dec.prefill_chunked([float(t) for t in prompt], True)
    assert res["passed"], res["error"]
    assert dec.current_length() == length
    V = cfg["vocabulary"]
    gpu_logits = res["logits"].reshape(length, V)
    tables = [dec.kv_block_table(l) for l in range(cfg["layers"])]
    ref = OracleRequest(orc, cfg, m, cfg["capacity"] // P)
    ref_logits, ref_next = _oracle_chunks(orc, cfg, m, ref, tables, prompt, chunk)
    assert_f16_path(gpu_logits, ref_logits, what=f"{name} chunked prefill logits")
    _check_token(int(res["next_token_ids"][-1]), int(ref_next[-1]), ref_logits[-1],
                 f"{name} prefill token")
    for l in range(cfg["layers"]):
        got_k = dec.read_key_prefix(l).reshape(cfg["kv_heads"], length, cfg["head_dim"])
        assert_f16_path(got_k, ref.prefix(l, tables[l], length), what=f"{name} K layer {l}")
        got_v = dec.read_value_prefix(l).reshape(cfg["kv_heads"], length, cfg["head_dim"])
        assert_f16_path(got_v, ref.prefix(l, tables[l], length, keys=False),
                        what=f"{name} V layer {l}")
    # decode continues from the chunked cache
    token = int(res["next_token_ids"][-1])
    for step in range(3):
        out = dec.decode([float(token)], True)
        assert out["passed"], out["error"]
        tables = [dec.kv_block_table(l) for l in range(cfg["layers"])]
        lg, nxt = ref.step(token, length + step + 1, tables)
        assert_f16_path(out["logits"], lg, what=f"{name} decode {step} after chunked prefill")
        _check_token(int(out["next_token_ids"][0]), nxt, lg, f"{name} decode {step}")
        token = int(out["next_token_ids"][0])


def test_prefill_chunked_agrees_with_token_steps(host, orc, rt):
    """The same prompt through prefill() (one decode step per token) and
    prefillChunked() on one compiled decoder: same logits to the fp16-path
    tolerance, same greedy continuation."""
    cfg = CONFIGS["gqa4_d128"]
    m = _weights(orc, cfg, 21)
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    opts.prefill_chunk_size = 32
    dec, _ = host.compile_decoder_llm(rt, _workload(host, orc, cfg, m), opts)
    prompt = [float(t) for t in np.random.default_rng(22).integers(0, cfg["vocabulary"], 75)]
    steps = dec.prefill(prompt, True)
    assert steps["passed"], steps["error"]
    assert dec.reset() == ""
    chunked = dec.prefill_chunked(prompt, True)
    assert chunked["passed"], chunked["error"]
    assert_f16_path(chunked["logits"], steps["logits"], what="chunked vs stepped prefill")


def test_prefill_chunked_errors(host, orc, rt):
    cfg = CONFIGS["mha_d64"]
    m = _weights(orc, cfg, 31)
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    dec, _ = host.compile_decoder_llm(rt, _workload(host, orc, cfg, m), opts)
    r = dec.prefill_chunked([1.0, 2.0])
    assert not r["passed"] and "not compiled" in r["error"]
    opts.prefill_chunk_size = 16
    dec, _ = host.compile_decoder_llm(rt, _workload(host, orc, cfg, m), opts)
    assert dec.prefill_chunked([1.0, 2.0])["passed"]
    r = dec.prefill_chunked([3.0])
    assert not r["passed"] and "empty cache" in r["error"]
    assert dec.reset() == ""
    r = dec.prefill_chunked([float(cfg["vocabulary"])])
    assert not r["passed"] and "vocabulary" in r["error"]
    assert dec.current_length() == 0
    r = dec.prefill_chunked([1.0] * (cfg["capacity"] + 1))
    assert not r["passed"] and "capacity" in r["error"]


def test_chunked_prefill_executor_direct(host, orc, rt):
    """The executor over shared pools: a prompt split at an arbitrary point
    (start > 0 with a partial first page) gives the oracle's logits."""
    cfg = CONFIGS["serve"]
    m = _weights(orc, cfg, 41)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    pools = [host.create_kv_page_pool(rt, w.plan.kv_plan(), P, 8) for _ in range(cfg["layers"])]
    ex = host.create_chunked_prefill_executor(rt, model, pools, 32)
    assert ex.buckets() == [16, 32] and ex.chunk_size() == 32
    max_pages = ex.max_pages()
    states = [host.create_kv_cache_state(rt, w.plan.kv_plan(), pools[l], False)
              for l in range(cfg["layers"])]
    for state in states:
        assert state.stage_length(rt, 45) == ""
    tables = [s.page_table() + [-1] * (max_pages - len(s.page_table())) for s in states]
    prompt = np.random.default_rng(42).integers(0, cfg["vocabulary"], 45)
    ref = OracleRequest(orc, cfg, m, 8)
    got = []
    for s, e in ((0, 19), (19, 45)):
        r = ex.run([int(t) for t in prompt[s:e]], s, tables, True, True)
        assert r["passed"], r["error"]
        assert r["gpu_us"] > 0
        got.append(r["logits"].reshape(e - s, -1))
    ref_logits = []
    for s, e in ((0, 19), (19, 45)):
        t = np.full((cfg["layers"], e - s, max_pages), -1, np.int32)
        for l, table in enumerate(tables):
            t[l, :, :] = table
        lg, _ = orc.decoder_step(m, cfg, ref.k, ref.v, P, max_pages, t, prompt[s:e],
                                 np.arange(s, e) + 1)
        ref_logits.append(lg)
    assert_f16_path(np.concatenate(got), np.concatenate(ref_logits), what="executor logits")
    # a table without the pages the chunk needs is refused before any launch
    short = [t[:1] + [-1] * (max_pages - 1) for t in tables]
    r = ex.run([1] * 20, 10, short)
    assert not r["passed"] and "not allocated" in r["error"]


# ------------------------------------------------- several requests per chunk
@pytest.mark.parametrize("qh,kvh,d", [(8, 8, 128), (16, 4, 128), (4, 2, 64)])
def test_prefill_rows_several_requests(tmc, orc, torch, qh, kvh, d):
    """Three requests packed in one chunk, each from a tile boundary (tile =
    64 / group rows), with their own tables and starts: RoPE + append equals
    the per-row decode form bit for bit, attention equals the oracle's causal
    attention per request, and padding rows are left untouched."""
    group = qh // kvh
    tile = 64 // group
    p, cap = 16, 256
    max_pages = cap // p
    pages = 3 * max_pages + 4
    perm = np.random.default_rng(760).permutation(pages).astype(np.int32)
    tables = perm[:3 * max_pages].reshape(3, max_pages).copy()
    counts, starts = [tile + 5, 3, 2 * tile], [17, 0, 100]
    firsts, row = [], 0
    for i, c in enumerate(counts):
        firsts.append(row)
        row = row + c if i == 2 else -(-(row + c) // tile) * tile
    rows = row
    lengths = np.zeros(rows, np.int32)
    row_table = np.full(rows, -1, np.int32)
    for i, (f, c, s0) in enumerate(zip(firsts, counts, starts)):
        lengths[f:f + c] = s0 + np.arange(c) + 1
        row_table[f:f + c] = i
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos, sin = np.cos(pos * freq).astype(np.float32), np.sin(pos * freq).astype(np.float32)
    qkv = orc.f16(normal(761, (rows, (qh + 2 * kvh) * d)))
    pool0 = orc.f16(normal(762, (pages, kvh, p, d)))
    act = torch.tensor([rows], dtype=torch.int32, device="cuda")
    # RoPE + append: row-table form vs per-row decode form
    outs = []
    for form in ("rows", "decode"):
        kp, vp = dev_f16(pool0), dev_f16(pool0.copy())
        q_out = torch.full((rows, qh * d), float("nan"), dtype=torch.float16, device="cuda")
        if form == "rows":
            tmc.prefill_rope_append_rows(dev_f16(qkv), dev(cos), dev(sin), dev(lengths),
                                         dev(tables), dev(row_table), act, q_out, kp, vp, rows, qh,
                                         kvh, d, cap, p, max_pages)
        else:
            per_row = np.where(row_table[:, None] >= 0, tables[np.maximum(row_table, 0)], -1)
            tmc.decode_rope_append(dev_f16(qkv), dev(cos), dev(sin), dev(lengths),
                                   dev(per_row.astype(np.int32)), act, q_out, kp, vp, rows, qh, kvh,
                                   d, cap, p, max_pages)
        torch.cuda.synchronize()
        outs.append((bits(q_out), bits(kp), bits(vp), q_out, kp, vp))
    for a, b in zip(outs[0][:3], outs[1][:3]):
        assert np.array_equal(a, b)
    # attention over the pools the append wrote
    q_out, kp, vp = outs[0][3:]
    ctx = torch.full((rows, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.prefill_attention_rows(q_out, kp, vp, dev(lengths), dev(tables), dev(row_table), act, ctx,
                               rows, qh, kvh, d, p, max_pages, kvh * p * d, p * d)
    torch.cuda.synchronize()
    got = values(ctx)
    k_np, v_np = bits(kp).reshape(pages, kvh, p, d), bits(vp).reshape(pages, kvh, p, d)
    q_np = bits(q_out)
    padding = row_table < 0
    assert np.isnan(got[padding]).all()
    for i, (f, c, s0) in enumerate(zip(firsts, counts, starts)):
        ref, written = orc.causal_prefill_attention(q_np[f:f + c], k_np, v_np, F16, qh, kvh, d, p,
                                                    kvh * p * d, p * d, tables[i], max_pages,
                                                    s0 + c, c)
        assert written.all()
        assert_f16_path(got[f:f + c], ref, what=f"request {i} rows")


def test_chunked_prefill_run_batch_matches_single_requests(host, orc, rt):
    """runBatch of three requests' segments (one split across two chunks)
    gives the next tokens, last-row logits and caches that single-request
    chunks give."""
    cfg = CONFIGS["serve"]
    m = _weights(orc, cfg, 71)
    w = _workload(host, orc, cfg, m)
    model = host.create_model_resources(rt, w)
    kv = w.plan.kv_plan()
    V = cfg["vocabulary"]
    prompts = [np.random.default_rng(72 + i).integers(0, V, n) for i, n in enumerate((21, 7, 40))]

    def run(batched):
        pools = [host.create_kv_page_pool(rt, kv, P, 16) for _ in range(cfg["layers"])]
        ex = host.create_chunked_prefill_executor(rt, model, pools, 64, 4 if batched else 1)
        states = [[host.create_kv_cache_state(rt, kv, pool, False) for pool in pools]
                  for _ in prompts]

        def segment(i, start, count):
            for s in states[i]:
                assert s.stage_length(rt, start + count) == ""
            tables = [s.page_table() + [-1] * (ex.max_pages() - len(s.page_table()))
                      for s in states[i]]
            return ([int(t) for t in prompts[i][start:start + count]], start, tables)

        def commit(i, length):
            for s in states[i]:
                s.commit_length(length)

        nxt, logits = {}, {}
        if batched:
            assert ex.tile_rows() == 32 and ex.maximum_requests() == 4
            # chunk 1: request 0 (21 rows, padded to 32) and request 1 (7)
            first = [segment(0, 0, 21), segment(1, 0, 7)]
            assert ex.packed_rows([21, 7]) == 39
            out = ex.run_batch(first, True)
            assert out["passed"], out["error"]
            commit(0, 21)
            commit(1, 7)
            ids = out["next_token_ids"]
            nxt[0], nxt[1] = ids[20], ids[27]
            logits[0], logits[1] = out["logits"][:V], out["logits"][V:]
            second = [segment(2, 0, 30)]
            out = ex.run_batch(second, False)
            assert out["passed"], out["error"]
            commit(2, 30)
            third = [segment(2, 30, 10)]
            out = ex.run_batch(third, True)
            assert out["passed"], out["error"]
            commit(2, 40)
            nxt[2], logits[2] = out["next_token_ids"][-1], out["logits"]
        else:
            for i, prompt in enumerate(prompts):
                done = 0
                while done < len(prompt):
                    c = min(64, len(prompt) - done)
                    tokens, start, tables = segment(i, done, c)
                    out = ex.run(tokens, start, tables, True)
                    assert out["passed"], out["error"]
                    commit(i, done + c)
                    done += c
                nxt[i], logits[i] = out["next_token_ids"][-1], out["logits"][-V:]
        caches = [[s.read_key_prefix() for s in st] for st in states]
        return nxt, logits, caches

    n1, l1, c1 = run(False)
    n2, l2, c2 = run(True)
    for i in range(3):
        assert_f16_path(l2[i], l1[i], what=f"request {i} last-row logits")
        if n1[i] != n2[i]:
            top = np.sort(l1[i])[-2:]
            assert top[1] - top[0] <= 2e-2
        for a, b in zip(c1[i], c2[i]):
            assert_f16_path(b, a, what=f"request {i} keys")
