"""Pins the CPU oracle (oracle/tmc_oracle.c) against the golden vectors that
tests/golden/make_golden.py wrote from the reference GraphReference, and
against closed forms for what the vectors leave open."""
import numpy as np
import pytest

F16, F32, BF16, I32 = 0, 1, 2, 3


def close(a, b, rel=1e-12):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    scale = max(1.0, float(np.max(np.abs(b)))) if b.size else 1.0
    return np.allclose(a, b, rtol=rel, atol=rel * scale, equal_nan=True)


def test_store_f16_matches_reference(orc, golden):
    x = golden["store_in"]
    bits = orc.f16(x)
    got = orc.f16_values(bits)
    exp = golden["store_f16"]
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    m = ~np.isnan(exp)
    assert np.array_equal(got[m].view(np.uint32), exp[m].view(np.uint32))


def test_store_f16_is_ties_away_not_rne(orc):
    # 1 + 2^-11 is exactly halfway between 1 and 1 + 2^-10.
    assert orc.f16_values(orc.f16([1.0 + 2.0 ** -11]))[0] == np.float32(1.0 + 2.0 ** -10)
    assert np.float16(np.float32(1.0 + 2.0 ** -11)) == np.float16(1.0)  # numpy RNE differs
    # off-tie values agree with IEEE RNE everywhere
    rng = np.random.default_rng(1)
    x = rng.standard_normal(100000).astype(np.float32)
    x = x[(x.view(np.uint32) & 0x1FFF) != 0x1000]  # drop exact ties of normal fp16 range
    got = orc.f16_values(orc.f16(x))
    assert np.array_equal(got, x.astype(np.float16).astype(np.float32))


def test_f16_decode_exhaustive_roundtrip(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = orc.f16_values(bits)
    ref = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(vals), np.isnan(ref))
    m = ~np.isnan(ref)
    assert np.array_equal(vals[m].view(np.uint32), ref[m].view(np.uint32))
    back = orc.f16(vals[m])
    assert np.array_equal(back, bits[m])


def test_store_other_dtypes(orc, golden):
    x = golden["store_in"]
    assert close(orc.store(x, F32), golden["store_f32"])
    assert close(orc.store(x, BF16), golden["store_bf16"])  # bf16 not rounded by storeValue
    assert np.array_equal(orc.store(golden["store_i32_in"], I32), golden["store_i32"])


def test_bf16_upload_is_rne(orc):
    import torch
    x = np.random.default_rng(3).standard_normal(10000).astype(np.float32)
    got = orc.decode(orc.encode(x, BF16), BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("name", ["rms_1x4096", "rms_3x4097", "rms_3x4097_e6", "rms_f16_1x257",
                                  "rms_f16_4x512"])
def test_rmsnorm_golden(orc, golden, name):
    dtype, eps = golden[f"{name}_meta"]
    dtype = int(dtype)
    x, w = golden[f"{name}_x"], golden[f"{name}_w"]
    if dtype == F16:
        out = orc.rmsnorm(orc.f16(x), orc.f16(w), F16, float(eps))
    else:
        out = orc.rmsnorm(x, w, F32, float(eps))
    assert close(out, golden[f"{name}_out"])


@pytest.mark.parametrize("name", ["addrms_3x4097", "addrms_f16_2x257", "addrms_f16_3x4096"])
def test_add_rmsnorm_golden(orc, golden, name):
    dtype = int(golden[f"{name}_dtype"][0])
    x, r, w = golden[f"{name}_x"], golden[f"{name}_r"], golden[f"{name}_w"]
    enc = (lambda a: orc.f16(a)) if dtype == F16 else (lambda a: np.asarray(a, np.float32))
    if dtype == F32:
        r = np.broadcast_to(r, x.shape)
    s, out = orc.add_rmsnorm(enc(x), enc(r), enc(w), dtype, 1e-6)
    assert np.array_equal(s, golden[f"{name}_sum"])
    assert close(out, golden[f"{name}_out"])


def test_linear_golden_matmul_on_transposed_weight(orc, golden):
    a, b = golden["mm_f32_a"], golden["mm_f32_b"]
    assert close(orc.linear(a, np.ascontiguousarray(b.T), F32), golden["mm_f32_out"])
    a, b = golden["mm_f16_a"], golden["mm_f16_b"]
    y = orc.linear(orc.f16(a), orc.f16(np.ascontiguousarray(b.T)), F16)
    assert close(y, golden["mm_f16_out"])


def test_linear_identity_and_basis(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    xb = orc.f16(x)
    eye = orc.f16(np.eye(64, dtype=np.float32))
    assert np.array_equal(orc.linear(xb, eye, F16).astype(np.float32), orc.f16_values(xb))
    # a transposed operand would swap rows/cols: pick a non-symmetric W
    w = np.zeros((5, 64), np.float32)
    w[2, 7] = 1.0
    y = orc.linear(xb, orc.f16(w), F16)
    assert np.all(y[:, [0, 1, 3, 4]] == 0) and np.array_equal(y[:, 2].astype(np.float32),
                                                             orc.f16_values(xb)[:, 7])


@pytest.mark.parametrize("name,dtype", [("silu_f32", F32), ("silu_f16", F16)])
def test_silu_mul_golden(orc, golden, name, dtype):
    gt, up = golden[f"{name}_g"], golden[f"{name}_u"]
    enc = (lambda a: orc.f16(a)) if dtype == F16 else (lambda a: np.asarray(a, np.float32))
    assert close(orc.silu_mul(enc(gt), enc(up), dtype), golden[f"{name}_out"])


def test_gated_mlp_is_composition(orc):
    rng = np.random.default_rng(9)
    x = orc.f16(rng.standard_normal((2, 64)))
    wg = orc.f16(rng.standard_normal((32, 64)) * 0.1)
    wu = orc.f16(rng.standard_normal((32, 64)) * 0.1)
    g = orc.store(orc.linear(x, wg, F16), F16)
    u = orc.store(orc.linear(x, wu, F16), F16)
    expect = orc.silu_mul(orc.f16(g), orc.f16(u), F16)
    assert close(orc.gated_mlp(x, wg, wu, F16), expect)


def test_rope_golden_and_norm(orc, golden):
    x, cos, sin = golden["rope_x"], golden["rope_cos"], golden["rope_sin"]
    out = orc.rope(x, cos, sin, F32, 2, 8, np.arange(3))
    assert close(out, golden["rope_out"])
    pairs = out.reshape(-1, 2)
    xin = x.astype(np.float64).reshape(-1, 2)
    assert np.allclose(np.hypot(pairs[:, 0], pairs[:, 1]), np.hypot(xin[:, 0], xin[:, 1]),
                       rtol=1e-6)


def test_attention_golden(orc, golden):
    q, k, v = golden["attn_q"], golden["attn_k"], golden["attn_v"]
    pairs, length, d, _ = golden["attn_meta"]
    pairs, length, d = int(pairs), int(length), int(d)
    # contiguous oracle: batch=1, q_heads=kv_heads=pairs, capacity=length
    out = orc.decode_attention(q.reshape(1, pairs * d), k.reshape(-1), v.reshape(-1), F32,
                               pairs, pairs, d, length, length)
    # The reference chain stores scores, scaled scores and probabilities as fp32
    # graph values; the oracle keeps them in double, so agreement is to fp32
    # rounding (a dropped term, a wrong scale or index is off by far more).
    assert close(out.reshape(-1), golden["attn_out"], rel=2e-6)


def test_attention_closed_forms(orc):
    rng = np.random.default_rng(11)
    d, cap = 16, 8
    q = orc.f16(rng.standard_normal((1, 2 * d)))
    k = orc.f16(rng.standard_normal((1, 1, cap, d)))
    v = orc.f16(rng.standard_normal((1, 1, cap, d)))
    # valid = 1 -> output is V[0] for every query head (GQA 2:1)
    out = orc.decode_attention(q, k, v, F16, 2, 1, d, cap, 1)
    v0 = orc.f16_values(v.reshape(cap, d)[0])
    assert np.allclose(out.reshape(2, d), v0[None, :], atol=1e-12)
    # equal keys -> uniform softmax -> mean of V
    k_same = np.broadcast_to(k.reshape(cap, d)[:1], (cap, d)).copy()
    out = orc.decode_attention(q, k_same, v, F16, 2, 1, d, cap, 5)
    mean = orc.f16_values(v.reshape(cap, d)[:5]).astype(np.float64).mean(axis=0)
    assert np.allclose(out.reshape(2, d), mean[None, :], atol=1e-12)


def test_paged_attention_matches_contiguous_through_tables(orc, golden):
    rng = np.random.default_rng(13)
    d, qh, kvh, p, pages, valid = 16, 4, 2, 4, 10, 13
    pool_k = orc.f16(rng.standard_normal((pages, kvh, p, d)))
    pool_v = orc.f16(rng.standard_normal((pages, kvh, p, d)))
    table = np.array([7, 2, 9, 0], np.int32)  # ceil(13/4) = 4 pages
    q = orc.f16(rng.standard_normal((1, qh * d)))
    out, written = orc.paged_attention(q, pool_k, pool_v, F16, qh, kvh, d, p, kvh * p * d, p * d,
                                       table[None, :], 4, [valid], 1)
    assert written.all()
    # gather the logical cache with the reference Gather semantics and compare
    gt = golden["gather_table"]
    assert close(gt[golden["gather_idx"].astype(int)], golden["gather_out"])
    cont_k = pool_k[table].transpose(1, 0, 2, 3).reshape(1, kvh, 4 * p, d)
    cont_v = pool_v[table].transpose(1, 0, 2, 3).reshape(1, kvh, 4 * p, d)
    ref = orc.decode_attention(q, cont_k, cont_v, F16, qh, kvh, d, 4 * p, valid)
    assert close(out, ref)
    # a negative page inside the valid range suppresses the write
    bad = table.copy()
    bad[2] = -1
    _, written = orc.paged_attention(q, pool_k, pool_v, F16, qh, kvh, d, p, kvh * p * d, p * d,
                                     bad[None, :], 4, [valid], 1)
    assert not written.any()


def test_causal_prefill_attention_is_masked_softmax(orc):
    """The causal chunk rule (query r of a chunk of S attends valid - S + r + 1
    positions) against textbook causal attention written independently here:
    softmax(Q K^T / sqrt(D) + M) V with M = -inf above the diagonal shifted by
    the tokens before the chunk (GQA 4:2, pages out of order, a 3-token
    prefix).  The last row of a chunk is the decode rule (valid positions),
    and a chunk of one is a decode step."""
    rng = np.random.default_rng(17)
    d, qh, kvh, p, pages = 16, 4, 2, 4, 6
    start, chunk = 3, 9
    valid = start + chunk
    pool_k = orc.f16(rng.standard_normal((pages, kvh, p, d)))
    pool_v = orc.f16(rng.standard_normal((pages, kvh, p, d)))
    table = np.array([4, 1, 5, 0], np.int32)  # 12 positions
    q = orc.f16(rng.standard_normal((chunk, qh * d)))
    out, written = orc.causal_prefill_attention(q, pool_k, pool_v, F16, qh, kvh, d, p,
                                                kvh * p * d, p * d, table, 4, valid, chunk)
    assert written.all()
    kf = orc.f16_values(pool_k)[table].transpose(1, 0, 2, 3).reshape(kvh, 4 * p, d)[:, :valid]
    vf = orc.f16_values(pool_v)[table].transpose(1, 0, 2, 3).reshape(kvh, 4 * p, d)[:, :valid]
    qf = orc.f16_values(q).reshape(chunk, qh, d).astype(np.float64)
    mask = np.arange(valid)[None, :] <= (start + np.arange(chunk))[:, None]  # [chunk, valid]
    expect = np.empty((chunk, qh, d))
    for h in range(qh):
        s = qf[:, h, :] @ kf[h // (qh // kvh)].T.astype(np.float64) / np.sqrt(d)
        s = np.where(mask, s, -np.inf)
        w = np.exp(s - s.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        expect[:, h, :] = w @ vf[h // (qh // kvh)].astype(np.float64)
    # the oracle stores outputs in fp16, the textbook form is exact
    assert np.max(np.abs(out.reshape(chunk, qh, d) - expect)) <= 2e-3 * max(1.0, np.abs(expect).max())
    last, _ = orc.paged_attention(q[-1:], pool_k, pool_v, F16, qh, kvh, d, p, kvh * p * d, p * d,
                                  table[None, :], 4, [valid], 1)
    assert close(out[-1:], last)
    one, _ = orc.causal_prefill_attention(q[:1], pool_k, pool_v, F16, qh, kvh, d, p, kvh * p * d,
                                          p * d, table, 4, start + 1, 1)
    assert close(one, out[:1])


def test_argmax_rules(orc):
    x = np.array([[1.0, 3.0, 3.0, 2.0], [np.nan, 0.5, np.nan, 0.5],
                  [-np.inf, -np.inf, -np.inf, -np.inf], [np.nan] * 4], np.float32)
    assert list(orc.argmax(x)) == [1, 1, 0, -1]


def test_compare_golden(orc, golden):
    a, r = golden["cmp_actual"], golden["cmp_ref"]
    for key, sel, atol, rtol in (("cmp_out_a", [0, 1, 2], 1e-3, 1e-3),
                                 ("cmp_out_b", [0, 1, 2, 3, 4], 1e-3, 1e-3),
                                 ("cmp_out_c", [0, 1, 4], 2e-3, 0.0)):
        ok, worst, mism = orc.compare(a[sel], r[sel], atol, rtol)
        exp = golden[key]
        assert ok == bool(exp[0]) and mism == int(exp[2])
        assert worst == exp[1] or (np.isinf(worst) and np.isinf(exp[1]))


def test_append_maps_are_bit_copies(orc):
    rng = np.random.default_rng(17)
    b, h, d, s, cap, p = 1, 2, 4, 3, 8, 2
    inp = rng.integers(0, 65535, size=b * s * h * d, dtype=np.uint16)
    cache = np.zeros(b * h * cap * d, np.uint16)
    out = orc.append_contiguous(inp, cache, b, h, d, s, cap, False, 5)
    view = out.reshape(b, h, cap, d)
    tok = inp.reshape(b, s, h, d)
    for t in range(s):
        assert np.array_equal(view[0, :, 2 + t, :], tok[0, t])
    assert np.count_nonzero(out) == np.count_nonzero(inp)
    # out-of-range valid length is a no-op
    assert np.array_equal(orc.append_contiguous(inp, cache, b, h, d, s, cap, False, 9), cache)
    table = np.array([3, 1, 0, 2], np.int32)
    pool = np.zeros(4 * b * h * p * d, np.uint16)
    out = orc.append_paged(inp, pool, b, h, d, s, cap, p, False, 5, table)
    pv = out.reshape(4, b, h, p, d)
    for t in range(s):
        pos = 2 + t
        assert np.array_equal(pv[table[pos // p], 0, :, pos % p, :], tok[0, t])


@pytest.mark.parametrize("head_major", [False, True])
def test_append_serving_places_each_row_through_its_table(orc, head_major):
    """tmco_append_serving (emitServingPagedCacheAppend,
    DecoderLLMMetalEmitter.cpp:314-373) pinned by tagged values: every input
    element carries its own (row, head, column) as its bits, so each written
    pool element names where it came from.  Written elements must be exactly
    those of the rows below active_count whose length lies in [1, capacity]
    and whose page entry for position length - 1 is present; each sits in
    page table[row][(length - 1) / page_size], head slab h, slot
    (length - 1) % page_size, column c ([page][heads][page_size][head_dim]);
    reading that position back through the row's table returns the row; and
    nothing else in the pool changes."""
    rng = np.random.default_rng(21)
    rows, heads, d, p, cap = 7, 3, 4, 4, 16
    max_pages = cap // p
    pages = rows * max_pages + 2
    hidden = heads * d
    tags = np.arange(1, rows * hidden + 1, dtype=np.uint16)  # row-major tag r * hidden + f + 1
    if head_major:  # [row][head][d]: the same element order for this layout
        inp = tags.reshape(rows, heads, d).copy().ravel()
    else:
        inp = tags.copy()
    tables = rng.permutation(pages)[:rows * max_pages].astype(np.int32).reshape(rows, max_pages)
    lengths = np.array([1, 5, cap, 0, cap + 1, 9, 3], np.int32)
    tables[5, (9 - 1) // p] = -1  # the target page of row 5 is missing
    active = 6  # row 6 is past the active count
    pool = np.zeros(pages * heads * p * d, np.uint16)
    out = orc.append_serving(inp, pool, rows, heads, d, cap, p, head_major, lengths, tables, active)
    view = out.reshape(pages, heads, p, d)
    expected_rows = [r for r in range(rows)
                     if r < active and 1 <= lengths[r] <= cap
                     and tables[r, (lengths[r] - 1) // p] >= 0]
    assert expected_rows == [0, 1, 2]
    written = np.argwhere(view != 0)
    assert len(written) == len(expected_rows) * hidden
    for page, h, slot, c in written:
        tag = int(view[page, h, slot, c]) - 1
        r, f = divmod(tag, hidden)
        assert r in expected_rows and divmod(f, d) == (h, c)
        pos = int(lengths[r]) - 1
        assert page == tables[r, pos // p] and slot == pos % p
    for r in expected_rows:  # the row read back through its own table
        pos = int(lengths[r]) - 1
        got = view[tables[r, pos // p], :, pos % p, :].ravel()
        assert np.array_equal(got, tags[r * hidden:(r + 1) * hidden])
