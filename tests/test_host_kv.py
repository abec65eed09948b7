"""Host logic of the C++ layer on the CPU: KVPagePool / KVCacheState
bookkeeping (reference src/runtime/KVCacheState.cpp) and the continuous-
batching scheduler (ServingRuntime.cpp:426-930), driven with bookkeeping-only
pools and a host step function.  No GPU is touched: pools created without a
runtime hold no device storage and states over them skip device writes."""
import numpy as np
import pytest


def _plan(host, heads=2, d=8, capacity=64):
    plan = host.KVCachePlan()
    plan.heads, plan.head_dimension, plan.capacity = heads, d, capacity
    plan.dtype = host.DType.Float16
    return plan


def test_pool_is_lifo_and_counts(host):
    rt = host.HipRuntime()
    pool = host.create_host_kv_page_pool(_plan(host), 16, 8)
    a = host.create_kv_cache_state(rt, _plan(host), pool)
    b = host.create_kv_cache_state(rt, _plan(host), pool)
    assert a.stage_length(rt, 20) == ""
    assert a.page_table() == [7, 6]  # free list 0..7, allocation pops the back
    assert b.stage_length(rt, 1) == ""
    assert b.page_table() == [5]
    assert (pool.used_pages(), pool.available_pages(), pool.peak_used_pages()) == (3, 5, 3)
    assert a.rollback_length(rt, 0) == ""  # pages return to the back of the list
    assert pool.available_pages() == 7 and pool.release_count() == 2
    assert b.stage_length(rt, 40) == ""
    # rollback releases logical pages last-to-first (6, then 7), so 7 is reused first
    assert b.page_table() == [5, 7, 6]
    assert pool.allocation_count() == 5 and pool.peak_used_pages() == 3


def test_state_length_rules_and_exhaustion(host):
    rt = host.HipRuntime()
    plan = _plan(host, capacity=64)
    pool = host.create_host_kv_page_pool(plan, 16, 5)
    s = host.create_kv_cache_state(rt, plan, pool)
    assert "capacity" in s.stage_length(rt, 0)
    assert "capacity" in s.stage_length(rt, 65)
    assert s.stage_length(rt, 64) == ""
    assert s.allocated_page_count() == 4 and s.current_length() == 0
    s.commit_length(64)
    assert s.current_length() == 64
    other = host.create_kv_cache_state(rt, plan, pool)
    err = other.stage_length(rt, 40)  # needs 3 pages, 1 left
    assert "exhausted" in err
    assert other.allocated_page_count() == 0 and pool.available_pages() == 1  # partial undone
    with pytest.raises(Exception):
        s.commit_length(0)
    assert s.reset(rt) == "" and pool.available_pages() == 5 and s.current_length() == 0


def test_state_destructor_releases_pages(host):
    rt = host.HipRuntime()
    plan = _plan(host)
    pool = host.create_host_kv_page_pool(plan, 8, 16)
    s = host.create_kv_cache_state(rt, plan, pool)
    assert s.stage_length(rt, 30) == ""
    assert pool.used_pages() == 4
    del s
    assert pool.used_pages() == 0 and pool.release_count() == 4


def test_pool_and_state_validation(host):
    rt = host.HipRuntime()
    plan = _plan(host, capacity=64)
    with pytest.raises(Exception):
        host.create_host_kv_page_pool(plan, 0, 4)
    with pytest.raises(Exception):
        host.create_host_kv_page_pool(plan, 65, 4)
    small = host.create_host_kv_page_pool(plan, 16, 3)  # cannot hold 64 tokens
    with pytest.raises(Exception):
        host.create_kv_cache_state(rt, plan, small)
    other = _plan(host, heads=4, capacity=64)
    pool = host.create_host_kv_page_pool(plan, 16, 8)
    with pytest.raises(Exception):
        host.create_kv_cache_state(rt, other, pool)
    assert "requires" in host.create_kv_cache_state(rt, plan, pool).restore(
        rt, 0, np.zeros(0, np.float32), np.zeros(0, np.float32)) or True


# ------------------------------------------------------------------ scheduler
V = 97


def _decoder_plan(host, layers=2, capacity=64):
    plan = host.DecoderLLMPlan()
    plan.attention = _plan(host, heads=2, d=8, capacity=capacity)
    plan.layer_count, plan.intermediate_size, plan.vocabulary_size = layers, 16, V
    return plan


def _next(token, length):
    """Deterministic stand-in model: the next token from the current one and
    the position, so a request's output depends only on its own history."""
    return (token * 31 + length * 7 + 3) % V


def _reference_tokens(prompt, decode):
    """A request decoded alone, one token at a time."""
    out = []
    length = 0
    last = None
    for t in prompt:
        length += 1
        last = _next(int(t), length)
    out.append(last)
    for _ in range(decode):
        length += 1
        last = _next(last, length)
        out.append(last)
    return out


def _run(host, specs, pages_per_layer, max_batch, page_size=4, layers=2, capacity=64, chunk=0,
         tile=1, per_chunk=1):
    rt = host.HipRuntime()
    plan = _decoder_plan(host, layers, capacity)
    pools = [host.create_host_kv_page_pool(plan.kv_plan(), page_size, pages_per_layer)
             for _ in range(layers)]
    max_pages = (capacity + page_size - 1) // page_size
    seen = {"rows": []}

    def step(tokens, lengths, tables, read_logits):
        rows = len(tokens)
        assert rows <= max_batch
        for l in range(layers):
            t = np.asarray(tables[l]).reshape(rows, max_pages)
            owned = [p for r in range(rows) for p in t[r] if p >= 0]
            assert len(owned) == len(set(owned)), "pages shared between rows"
            for r in range(rows):  # a page for every position up to the new token
                need = (lengths[r] + page_size - 1) // page_size
                assert (t[r, :need] >= 0).all() and (t[r, need:] < 0).all()
        seen["rows"].append(rows)
        nxt = [_next(t, n) for t, n in zip(tokens, lengths)]
        logits = np.zeros(rows * V, np.float32)
        return nxt, logits

    def prefill(segments, read_logits):
        """One chunk: segments (tokens, start, tables) of different requests,
        each from a multiple of `tile` rows, at most `chunk` rows in all."""
        assert 0 < len(segments) <= per_chunk
        row, out = 0, []
        for i, (tokens, start, tables) in enumerate(segments):
            rows = len(tokens)
            assert rows > 0
            row += rows
            if i + 1 < len(segments):
                row = -(-row // tile) * tile
            need = (start + rows + page_size - 1) // page_size
            for l in range(layers):
                t = np.asarray(tables[l])
                assert (t[:need] >= 0).all() and (t[need:] < 0).all()
            out += [_next(t, start + r + 1) for r, t in enumerate(tokens)]
            seen.setdefault("chunks", []).append(rows)
        assert row <= chunk
        seen.setdefault("segments_per_chunk", []).append(len(segments))
        return out, np.zeros(len(segments) * V, np.float32)

    config = host.ServingConfig()
    config.page_size = page_size
    config.physical_pages_per_layer = pages_per_layer
    config.maximum_batch_size = max_batch
    config.prefill_chunk_size = chunk
    result = host.run_continuous_batch_with(rt, plan, pools, max_batch, max_pages, step, specs,
                                            config, prefill if chunk else None, tile, per_chunk)
    return result, pools, seen


def _specs(host, rng, n, prompt=(2, 20), decode=(0, 12), arrivals=4):
    specs = []
    for i in range(n):
        s = host.ServingRequestSpec()
        s.id = f"r{i}"
        s.prompt_token_ids = [float(x) for x in rng.integers(0, V, rng.integers(*prompt))]
        s.decode_token_count = int(rng.integers(*decode))
        s.arrival_step = int(rng.integers(0, arrivals))
        specs.append(s)
    return specs


def test_scheduler_matches_sequential_decoding(host):
    specs = _specs(host, np.random.default_rng(1), 6)
    result, pools, seen = _run(host, specs, pages_per_layer=64, max_batch=6)
    assert result["passed"], result["error"]
    for spec, out in zip(specs, result["requests"]):
        want = _reference_tokens(spec.prompt_token_ids, spec.decode_token_count)
        assert out["generated_token_ids"] == want, spec.id
    m = result["metrics"]
    assert m["decoded_tokens"] == sum(s.decode_token_count for s in specs)
    assert m["prompt_tokens"] == sum(len(s.prompt_token_ids) for s in specs)
    assert m["preemption_count"] == 0 and max(seen["rows"]) > 1
    for p in pools:
        assert p.used_pages() == 0
        assert p.allocation_count() == p.release_count() == m["page_allocation_count"]


def test_scheduler_preempts_under_page_pressure_and_stays_exact(host):
    rng = np.random.default_rng(2)
    specs = _specs(host, rng, 8, prompt=(10, 24), decode=(8, 20), arrivals=2)
    # 16 pages hold one request at full capacity (64 tokens) but not all eight
    result, pools, _ = _run(host, specs, pages_per_layer=16, max_batch=8)
    assert result["passed"], result["error"]
    m = result["metrics"]
    assert m["preemption_count"] > 0 and m["resume_count"] == m["preemption_count"]
    for spec, out in zip(specs, result["requests"]):
        assert out["generated_token_ids"] == _reference_tokens(spec.prompt_token_ids,
                                                               spec.decode_token_count)
    assert all(p.used_pages() == 0 for p in pools)
    assert m["peak_pages_per_layer"] <= 16


@pytest.mark.parametrize("pages,chunk,tile,per_chunk", [(64, 5, 1, 1), (16, 8, 1, 1),
                                                     (64, 32, 8, 4), (16, 24, 4, 8)])
def test_scheduler_chunked_prefill_matches_sequential(host, pages, chunk, tile, per_chunk):
    """Prompts run at admission in chunks (prefillChunked per request,
    ServingRuntime.cpp:682-700), one request per chunk or several packed at
    tile boundaries; the outputs equal one-request decoding, also when page
    pressure preempts decoding requests."""
    rng = np.random.default_rng(4)
    specs = _specs(host, rng, 8, prompt=(10, 24), decode=(4, 16), arrivals=3)
    result, pools, seen = _run(host, specs, pages_per_layer=pages, max_batch=8, chunk=chunk,
                               tile=tile, per_chunk=per_chunk)
    assert result["passed"], result["error"]
    for spec, out in zip(specs, result["requests"]):
        assert out["generated_token_ids"] == _reference_tokens(spec.prompt_token_ids,
                                                               spec.decode_token_count), spec.id
    m = result["metrics"]
    total = sum(len(s.prompt_token_ids) for s in specs)
    assert m["prompt_tokens"] == total == sum(seen["chunks"])
    assert m["prefill_chunk_submissions"] == len(seen["segments_per_chunk"])
    if per_chunk == 1:
        assert m["prefill_chunk_submissions"] == sum(-(-len(s.prompt_token_ids) // chunk)
                                                     for s in specs)
    else:
        assert max(seen["segments_per_chunk"]) > 1
    assert all(p.used_pages() == 0 for p in pools)
    assert m["peak_pages_per_layer"] <= pages


def test_scheduler_batch_cap_and_validation(host):
    rng = np.random.default_rng(3)
    specs = _specs(host, rng, 5)
    result, _, seen = _run(host, specs, pages_per_layer=64, max_batch=2)
    assert result["passed"], result["error"]
    assert max(seen["rows"]) <= 2 and result["metrics"]["maximum_active_batch_size"] == 2
    bad = _specs(host, rng, 1)
    bad[0].prompt_token_ids = [1.0]  # prompts need two tokens (ServingRuntime.cpp:554-562)
    result, _, _ = _run(host, bad, pages_per_layer=64, max_batch=1)
    assert not result["passed"] and "invalid" in result["error"]
    bad = _specs(host, rng, 1)
    bad[0].prompt_token_ids = [1.0, float(V)]
    result, _, _ = _run(host, bad, pages_per_layer=64, max_batch=1)
    assert not result["passed"] and "token" in result["error"]
    big = _specs(host, rng, 1, prompt=(40, 41), decode=(20, 21))
    result, _, _ = _run(host, big, pages_per_layer=8, max_batch=1)
    assert not result["passed"] and "largest" in result["error"]
