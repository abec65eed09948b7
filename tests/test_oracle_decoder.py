"""The oracle's decoder step (tmco_decoder_step) against the composition of
the separately pinned oracle ops, in the order of the reference's decode
stage (DecoderLLMExecutor.cpp:322-849): embedding, RMSNorm, q/k/v linears,
RoPE, paged K/V append, paged attention, o linear, residual Add+RMSNorm,
gated MLP, down linear, residual add, final RMSNorm, LM head, argmax — every
output stored in fp16 before the next op reads it.  Each op used here is
pinned by the golden vectors of the compiled reference (test_oracle.py), so
this test pins the step's wiring: head grouping, residual order, rounding
points and page addressing."""
import numpy as np
import pytest

CFG = dict(layers=2, hidden=64, heads=4, head_dim=16, intermediate=96, vocabulary=50,
           capacity=32, epsilon=1e-6)
P = 4  # page size


def _model(orc, rng, kv_heads, vocabulary=CFG["vocabulary"]):
    H, I, V, D = CFG["hidden"], CFG["intermediate"], vocabulary, CFG["head_dim"]
    kv = kv_heads * D
    f16 = lambda a: orc.f16(np.asarray(a, np.float32))  # noqa: E731
    w = lambda *shape: f16(rng.standard_normal(shape) * 0.2)  # noqa: E731
    layers = []
    for _ in range(CFG["layers"]):
        layers.append(dict(input_norm=f16(rng.uniform(0.5, 1.5, H)), wq=w(H, H), wk=w(kv, H),
                           wv=w(kv, H), wo=w(H, H), post_norm=f16(rng.uniform(0.5, 1.5, H)),
                           wg=w(I, H), wu=w(I, H), wd=w(H, I)))
    pos = np.arange(CFG["capacity"], dtype=np.float64)[:, None]
    freq = 10000.0 ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    return dict(embedding=w(V, H), final_norm=f16(rng.uniform(0.5, 1.5, H)), lm_head=w(V, H),
                rope_cos=np.cos(pos * freq).astype(np.float32),
                rope_sin=np.sin(pos * freq).astype(np.float32), layers=layers)


def _composed_step(orc, m, kv_heads, kpools, vpools, tables, tokens, lengths):
    F16 = orc.F16
    H, D, NH, eps = CFG["hidden"], CFG["head_dim"], CFG["heads"], CFG["epsilon"]
    max_pages = CFG["capacity"] // P
    store = lambda x: orc.f16(np.asarray(x, np.float64).astype(np.float32))  # noqa: E731
    vals = orc.f16_values
    batch = len(tokens)
    cur = m["embedding"][tokens]
    pos = np.asarray(lengths) - 1
    for l, w in enumerate(m["layers"]):
        n = store(orc.rmsnorm(cur, w["input_norm"], F16, eps))
        q = store(orc.linear(n, w["wq"], F16))
        k = store(orc.linear(n, w["wk"], F16))
        v = store(orc.linear(n, w["wv"], F16))
        q = store(orc.rope(q, m["rope_cos"], m["rope_sin"], F16, NH, D, pos))
        k = store(orc.rope(k, m["rope_cos"], m["rope_sin"], F16, kv_heads, D, pos))
        t = tables[l]
        kpools[l][:] = orc.append_serving(k, kpools[l], batch, kv_heads, D, CFG["capacity"], P,
                                          False, lengths, t, batch)
        vpools[l][:] = orc.append_serving(v, vpools[l], batch, kv_heads, D, CFG["capacity"], P,
                                          False, lengths, t, batch)
        ctx, written = orc.paged_attention(q, kpools[l], vpools[l], F16, NH, kv_heads, D, P,
                                           kv_heads * P * D, P * D, t, max_pages, lengths, batch)
        assert written.all()
        ctx = store(ctx)
        o = store(orc.linear(ctx, w["wo"], F16))
        after, n2 = orc.add_rmsnorm(cur, o, w["post_norm"], F16, eps)
        after, n2 = orc.f16(after), store(n2)
        g = store(orc.gated_mlp(n2, w["wg"], w["wu"], F16))
        mlp = store(orc.linear(g, w["wd"], F16))
        cur = store(vals(after).astype(np.float64) + vals(mlp))
    n = store(orc.rmsnorm(cur, m["final_norm"], F16, eps))
    logits = orc.linear(n, m["lm_head"], F16).astype(np.float32)
    return logits, orc.argmax(logits)


@pytest.mark.parametrize("kv_heads", [4, 2])
def test_decoder_step_is_the_composition_of_pinned_ops(orc, kv_heads):
    rng = np.random.default_rng(77 + kv_heads)
    m = _model(orc, rng, kv_heads)
    cfg = dict(CFG, kv_heads=kv_heads)
    D, pages = CFG["head_dim"], 24
    max_pages = CFG["capacity"] // P
    perm = rng.permutation(pages).astype(np.int32)
    tables = np.full((CFG["layers"], 2, max_pages), -1, np.int32)
    for l in range(CFG["layers"]):  # disjoint pages per row, different per layer
        p = np.roll(perm, 5 * l)
        tables[l, 0, :max_pages // 2] = p[:max_pages // 2]
        tables[l, 1, :max_pages // 2] = p[max_pages // 2:max_pages]
    pool_shape = pages * kv_heads * P * D
    a_k = [np.zeros(pool_shape, np.uint16) for _ in range(CFG["layers"])]
    a_v = [np.zeros(pool_shape, np.uint16) for _ in range(CFG["layers"])]
    b_k = [p.copy() for p in a_k]
    b_v = [p.copy() for p in a_v]
    seq = rng.integers(0, CFG["vocabulary"], size=(2, 9))
    for step in range(9):
        tokens = seq[:, step].astype(np.int32)
        lengths = np.array([step + 1, step + 1], np.int32)
        if step >= 2:  # second row starts later: ragged lengths
            lengths[1] = step - 1
            tokens[1] = seq[1, step - 2]
        got_logits, got_tokens = orc.decoder_step(m, cfg, a_k, a_v, P, max_pages, tables, tokens,
                                                  lengths)
        want_logits, want_tokens = _composed_step(orc, m, kv_heads, b_k, b_v, tables, tokens,
                                                  lengths)
        np.testing.assert_allclose(got_logits, want_logits, rtol=1e-6, atol=1e-6)
        assert (got_tokens == want_tokens).all()
        for l in range(CFG["layers"]):
            assert (a_k[l] == b_k[l]).all() and (a_v[l] == b_v[l]).all()


def test_decoder_step_layer_limit_and_bad_inputs(orc):
    rng = np.random.default_rng(5)
    m = _model(orc, rng, 4)
    max_pages = CFG["capacity"] // P
    k = [np.zeros(32 * 4 * P * 16, np.uint16) for _ in range(2)]
    v = [x.copy() for x in k]
    tables = np.tile(np.arange(max_pages, dtype=np.int32), (2, 1, 1))
    with pytest.raises(ValueError):
        orc.decoder_step(m, CFG, k, v, P, max_pages, tables, np.array([CFG["vocabulary"]]),
                         np.array([1]))
    with pytest.raises(ValueError):
        orc.decoder_step(m, CFG, k, v, P, max_pages, tables, np.array([1]),
                         np.array([CFG["capacity"] + 1]))
    logits, _ = orc.decoder_step(m, CFG, k, v, P, max_pages, tables, np.array([3]), np.array([1]),
                                 layer_limit=1)
    assert not logits.any()  # the head runs only when every layer ran
    assert k[0].any() and not k[1].any()


@pytest.mark.parametrize("threads", [1, 4])
def test_decoder_step_row_blocks_threads_and_logits_from(orc, threads):
    """35 rows (two 16-row blocks of the blocked linear plus a 3-row tail),
    an odd vocabulary (a lone last output feature), 1 or 4 threads: the same
    values as the composition of pinned ops; rows before logits_from skip the
    LM head without changing the other rows' logits or any pool bit."""
    rng = np.random.default_rng(91)
    V, rows, kv_heads = 51, 35, 2
    m = _model(orc, rng, kv_heads, vocabulary=V)
    cfg = dict(CFG, kv_heads=kv_heads, vocabulary=V)
    D, max_pages = CFG["head_dim"], CFG["capacity"] // P
    pages = rows * 2
    tables = np.full((CFG["layers"], rows, max_pages), -1, np.int32)
    for l in range(CFG["layers"]):
        perm = rng.permutation(pages).astype(np.int32)
        tables[l, :, :2] = perm.reshape(rows, 2)
    size = pages * kv_heads * P * D
    pools = lambda: [np.zeros(size, np.uint16) for _ in range(CFG["layers"])]  # noqa: E731
    a_k, a_v, b_k, b_v, c_k, c_v = pools(), pools(), pools(), pools(), pools(), pools()
    tokens = rng.integers(0, V, rows).astype(np.int32)
    lengths = rng.integers(1, 2 * P + 1, rows).astype(np.int32)
    try:
        orc.set_threads(threads)
        got, got_tok = orc.decoder_step(m, cfg, a_k, a_v, P, max_pages, tables, tokens, lengths)
        part, part_tok = orc.decoder_step(m, cfg, c_k, c_v, P, max_pages, tables, tokens, lengths,
                                          logits_from=20)
    finally:
        orc.set_threads(1)
    want, want_tok = _composed_step(orc, m, kv_heads, b_k, b_v, tables, tokens, lengths)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    assert (got_tok == want_tok).all()
    for l in range(CFG["layers"]):
        assert (a_k[l] == b_k[l]).all() and (a_v[l] == b_v[l]).all()
        assert (c_k[l] == a_k[l]).all() and (c_v[l] == a_v[l]).all()
    assert not part[:20].any() and (part_tok[:20] == -1).all()
    np.testing.assert_array_equal(part[20:], got[20:])
    assert (part_tok[20:] == got_tok[20:]).all()


@pytest.mark.parametrize("threads", [1, 3])
def test_linear_values_equals_pinned_linear(orc, threads):
    """The blocked, threaded linear of the decode step gives the pinned
    tmco_linear's doubles bit for bit (rows 37: two 16-row blocks and a tail;
    an odd output count)."""
    rng = np.random.default_rng(17)
    x = orc.f16(rng.standard_normal((37, 96)).astype(np.float32))
    w = orc.f16((rng.standard_normal((51, 96)) * 0.1).astype(np.float32))
    try:
        orc.set_threads(threads)
        fast = orc.linear_values(x, w)
    finally:
        orc.set_threads(1)
    ref = orc.linear(x, w, orc.F16)
    assert np.array_equal(fast.view(np.uint64), np.asarray(ref, np.float64).view(np.uint64))
