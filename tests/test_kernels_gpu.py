"""GPU parity: every gfx950 kernel entry point against the CPU oracle on the
same seeded inputs, at BASELINE.json sizes where the oracle finishes in
seconds.  Calls go through the C ABI (libtmc_hip.so via ctypes)."""
import numpy as np
import pytest

from tests.helpers import (F16, F32, assert_f16_path, assert_f32_rel, bits, dev, dev_f16, normal,
                           uniform, values)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


# ---------------------------------------------------------------- config 1
def test_c1_rmsnorm_then_linear(tmc, orc, torch):
    """RMSNorm fp32 [1,4096] -> host fp16 cast -> GEMV fp16 W[4096,4096] -> fp32 y."""
    x = normal(101, (1, 4096))
    gamma = uniform(102, (4096,), 0.5, 1.5)
    w = orc.f16(normal(103, (4096, 4096), 0.02))
    xd, gd = dev(x), dev(gamma)
    yd = torch.empty_like(xd)
    tmc.rmsnorm(xd, gd, yd, 1e-6)
    torch.cuda.synchronize()
    ref_norm = orc.rmsnorm(x, gamma, F32, 1e-6)
    assert_f32_rel(values(yd), ref_norm, what="rmsnorm fp32")
    xh = orc.f16(values(yd))  # the host cast between the two graphs (ties away)
    out = torch.empty((1, 4096), dtype=torch.float32, device="cuda")
    tmc.gemv(dev_f16(xh), dev_f16(w), out)
    torch.cuda.synchronize()
    assert_f32_rel(values(out), orc.linear(xh, w, F16), what="gemv fp32 out")


@pytest.mark.parametrize("rows,width", [(3, 4097), (1, 4096), (2, 1), (5, 257)])
def test_rmsnorm_fp32_ragged_zero_and_tiny_rows(tmc, orc, torch, rows, width):
    x = normal(104, (rows, width))
    if rows > 1:
        x[0] = 0.0
        x[1] *= 1e-4
    gamma = uniform(105, (width,), 0.5, 1.5)
    y = torch.empty((rows, width), dtype=torch.float32, device="cuda")
    tmc.rmsnorm(dev(x), dev(gamma), y, 1e-6)
    torch.cuda.synchronize()
    assert_f32_rel(values(y), orc.rmsnorm(x, gamma, F32, 1e-6), what=f"rmsnorm {rows}x{width}")


@pytest.mark.parametrize("rows,width", [(1, 4096), (16, 4096), (1, 257)])
def test_rmsnorm_fp16(tmc, orc, torch, rows, width):
    x = orc.f16(normal(106, (rows, width)))
    gamma = orc.f16(uniform(107, (width,), 0.5, 1.5))
    y = torch.empty((rows, width), dtype=torch.float16, device="cuda")
    tmc.rmsnorm(dev_f16(x), dev_f16(gamma), y, 1e-6)
    torch.cuda.synchronize()
    assert_f16_path(values(y), orc.rmsnorm(x, gamma, F16, 1e-6), what="rmsnorm fp16")


@pytest.mark.parametrize("threads", [64, 128, 256, 512, 1024])
@pytest.mark.parametrize("variant", [0, 1])
def test_rmsnorm_threads_variants(tmc, orc, torch, threads, variant):
    """The RMSNorm tuner's candidates: every workgroup size, register-resident
    and two-pass, ragged fp32 rows and fp16 rows, plain and fused add."""
    for rows, width in ((3, 4097), (2, 4096), (1, 8)):
        x = normal(330, (rows, width))
        x[0] *= 1e-4
        gamma = uniform(331, (width,), 0.5, 1.5)
        y = torch.empty((rows, width), dtype=torch.float32, device="cuda")
        tmc.rmsnorm_threads(dev(x), dev(gamma), y, 1e-6, threads, variant)
        torch.cuda.synchronize()
        assert_f32_rel(values(y), orc.rmsnorm(x, gamma, F32, 1e-6),
                       what=f"rmsnorm t{threads} v{variant} {rows}x{width}")
    for rows, width in ((16, 4096), (3, 8200)):
        h = orc.f16(normal(332, (rows, width)))
        r = orc.f16(normal(333, (rows, width)))
        gamma = orc.f16(uniform(334, (width,), 0.5, 1.5))
        y = torch.empty((rows, width), dtype=torch.float16, device="cuda")
        tmc.rmsnorm_threads(dev_f16(h), dev_f16(gamma), y, 1e-6, threads, variant)
        s_out = torch.empty((rows, width), dtype=torch.float16, device="cuda")
        n_out = torch.empty((rows, width), dtype=torch.float16, device="cuda")
        tmc.add_rmsnorm_threads(dev_f16(r), dev_f16(h), dev_f16(gamma), s_out, n_out, 1e-6,
                                threads, variant)
        torch.cuda.synchronize()
        assert_f16_path(values(y), orc.rmsnorm(h, gamma, F16, 1e-6),
                        what=f"rmsnorm fp16 t{threads} v{variant}")
        ref_s, ref_n = orc.add_rmsnorm(r, h, gamma, F16, 1e-6)
        assert_f16_path(values(s_out), ref_s, what=f"residual sum t{threads} v{variant}")
        assert_f16_path(values(n_out), ref_n, what=f"add_rmsnorm t{threads} v{variant}")


def test_rmsnorm_threads_rejects_bad_workgroups(tmc, torch):
    x = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    for threads, variant in ((96, 0), (2048, 0), (256, 2)):
        with pytest.raises(tmc.TmcError):
            tmc.rmsnorm_threads(x, x[0], x, 1e-6, threads, variant)


# ---------------------------------------------------------------- GEMV family
@pytest.mark.parametrize("batch,k,n,out_dtype", [
    (1, 4096, 4096, F32), (1, 4096, 4096, F16), (2, 4096, 1024, F16), (3, 11008, 512, F32),
    (8, 4096, 4096, F16), (1, 4096, 32000, F32), (1, 11008, 4096, F32), (4, 136, 72, F32),
])
def test_gemv_fma_path(tmc, orc, torch, batch, k, n, out_dtype):
    x = orc.f16(normal(201, (batch, k)))
    w = orc.f16(normal(202, (n, k), 0.02))
    y = torch.empty((batch, n), dtype=torch.float32 if out_dtype == F32 else torch.float16,
                    device="cuda")
    tmc.gemv(dev_f16(x), dev_f16(w), y)
    torch.cuda.synchronize()
    ref = orc.linear(x, w, F16)
    if out_dtype == F32:
        assert_f32_rel(values(y), ref, what=f"gemv b{batch} k{k} n{n}")
    else:
        assert_f16_path(values(y), ref, what=f"gemv b{batch} k{k} n{n}")


@pytest.mark.parametrize("batch,k,n,out_dtype", [
    (16, 4096, 4096, F32), (16, 11008, 4096, F16), (9, 4096, 1000, F32), (33, 256, 72, F32),
    (64, 512, 48, F16), (1, 4096, 256, F32), (100, 128, 40, F32),
])
def test_skinny_gemm_mfma(tmc, orc, torch, batch, k, n, out_dtype):
    x = orc.f16(normal(203, (batch, k)))
    w = orc.f16(normal(204, (n, k), 0.02))
    y = torch.empty((batch, n), dtype=torch.float32 if out_dtype == F32 else torch.float16,
                    device="cuda")
    tmc.skinny_gemm(dev_f16(x), dev_f16(w), y)
    torch.cuda.synchronize()
    ref = orc.linear(x, w, F16)
    if out_dtype == F32:
        assert_f32_rel(values(y), ref, what=f"mfma b{batch} k{k} n{n}")
    else:
        assert_f16_path(values(y), ref, what=f"mfma b{batch} k{k} n{n}")


def test_gemv_unaligned_k_generic_path(tmc, orc, torch):
    x = orc.f16(normal(205, (2, 4097)))
    w = orc.f16(normal(206, (33, 4097), 0.02))
    y = torch.empty((2, 33), dtype=torch.float32, device="cuda")
    tmc.gemv(dev_f16(x), dev_f16(w), y)
    torch.cuda.synchronize()
    assert_f32_rel(values(y), orc.linear(x, w, F16), what="generic gemv")


def test_gemv_rejects_bad_arguments(tmc, torch):
    x = torch.zeros((1, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(tmc.TmcError):
        tmc.gemv(x, x, torch.zeros((1, 1), dtype=torch.int32, device="cuda"))


# ---------------------------------------------------------------- config 2
@pytest.mark.parametrize("batch", [1, 8])
def test_c2_fused_mlp_block(tmc, orc, torch, batch):
    h_, inter = 4096, 11008
    h = orc.f16(normal(201, (batch, h_)))
    r = orc.f16(normal(202, (batch, h_)))
    gamma = orc.f16(uniform(203, (h_,), 0.5, 1.5))
    wg = orc.f16(normal(204, (inter, h_), 0.02))
    wu = orc.f16(normal(205, (inter, h_), 0.02))
    wd = orc.f16(normal(206, (h_, inter), 0.02))
    s_d = torch.empty((batch, h_), dtype=torch.float16, device="cuda")
    n_d = torch.empty_like(s_d)
    g_d = torch.empty((batch, inter), dtype=torch.float16, device="cuda")
    y_d = torch.empty((batch, h_), dtype=torch.float32, device="cuda")
    tmc.add_rmsnorm(dev_f16(h), dev_f16(r), dev_f16(gamma), s_d, n_d, 1e-6)
    tmc.gate_up_silu(n_d, dev_f16(wg), dev_f16(wu), g_d)
    tmc.gemv(g_d, dev_f16(wd), y_d)
    torch.cuda.synchronize()
    # stage by stage on the GPU's own stage inputs
    s_ref, n_ref = orc.add_rmsnorm(h, r, gamma, F16, 1e-6)
    assert_f16_path(values(s_d), s_ref, what="residual sum")
    assert_f16_path(values(n_d), n_ref, what="add+rmsnorm")
    assert_f16_path(values(g_d), orc.gated_mlp(bits(n_d), wg, wu, F16), what="gate/up silu")
    assert_f32_rel(values(y_d), orc.linear(bits(g_d), wd, F16), what="down fp32")
    # end to end against the oracle chain
    n_chain = orc.f16(orc.store(n_ref, F16))
    g_chain = orc.f16(orc.store(orc.gated_mlp(n_chain, wg, wu, F16), F16))
    assert_f16_path(values(y_d), orc.linear(g_chain, wd, F16), what="mlp block end to end")


def test_gate_up_silu_batches_and_generic(tmc, orc, torch):
    for batch, hidden, inter in ((3, 256, 200), (16, 512, 64), (2, 100, 30)):
        x = orc.f16(normal(207, (batch, hidden)))
        wg = orc.f16(normal(208, (inter, hidden), 0.1))
        wu = orc.f16(normal(209, (inter, hidden), 0.1))
        out = torch.empty((batch, inter), dtype=torch.float16, device="cuda")
        tmc.gate_up_silu(dev_f16(x), dev_f16(wg), dev_f16(wu), out)
        torch.cuda.synchronize()
        assert_f16_path(values(out), orc.gated_mlp(x, wg, wu, F16),
                        what=f"gated mlp {batch}x{hidden}x{inter}")


def test_silu_mul_and_add(tmc, orc, torch):
    g = orc.f16(normal(210, (3, 11008)) * 4)
    u = orc.f16(normal(211, (3, 11008)))
    out = torch.empty((3, 11008), dtype=torch.float16, device="cuda")
    tmc.silu_mul(dev_f16(g), dev_f16(u), out)
    torch.cuda.synchronize()
    assert_f16_path(values(out), orc.silu_mul(g, u, F16), what="silu_mul fp16")
    # the 8-wide path (16-byte aligned, count % 8 == 0) and the one-element
    # path (a 2-byte-offset view) agree bit for bit
    gd, ud = dev_f16(g).reshape(-1), dev_f16(u).reshape(-1)
    one = torch.empty(gd.numel() - 1, dtype=torch.float16, device="cuda")
    tmc.silu_mul(gd[1:], ud[1:], one)
    torch.cuda.synchronize()
    assert torch.equal(out.reshape(-1)[1:], one)
    g32, u32 = normal(212, (4097,)) * 8, normal(213, (4097,))
    o32 = torch.empty(4097, dtype=torch.float32, device="cuda")
    tmc.silu_mul(dev(g32), dev(u32), o32)
    s = torch.empty(4097, dtype=torch.float32, device="cuda")
    tmc.add(dev(g32), dev(u32), s)
    torch.cuda.synchronize()
    assert_f32_rel(values(o32), orc.silu_mul(g32, u32, F32), what="silu_mul fp32")
    assert np.array_equal(values(s), (g32 + u32).astype(np.float32))


# ---------------------------------------------------------------- appends
@pytest.mark.parametrize("length", [128, 1024, 4095])
def test_c3_contiguous_append_bit_exact(tmc, orc, torch, length):
    heads, d, cap = 32, 128, 4096
    cache = orc.f16(normal(301, (1, heads, cap, d)))
    new = orc.f16(normal(304, (1, heads * d)))
    cache_d = dev_f16(cache)
    valid = torch.tensor([length + 1], dtype=torch.int32, device="cuda")
    tmc.kv_append(dev_f16(new), valid, cache_d, 1, 1, heads, d, cap, False)
    torch.cuda.synchronize()
    expect = orc.append_contiguous(new, cache.ravel(), 1, heads, d, 1, cap, False, length + 1)
    assert np.array_equal(bits(cache_d).ravel(), expect)


def test_append_rejects_out_of_range_valid(tmc, orc, torch):
    heads, d, cap = 4, 16, 8
    cache = orc.f16(normal(305, (1, heads, cap, d)))
    cache_d = dev_f16(cache)
    for bad in (0, cap + 1):
        valid = torch.tensor([bad], dtype=torch.int32, device="cuda")
        tmc.kv_append(dev_f16(orc.f16(normal(306, (1, heads * d)))), valid, cache_d, 1, 1, heads,
                      d, cap, False)
    torch.cuda.synchronize()
    assert np.array_equal(bits(cache_d), cache)


def test_paged_and_serving_append_bit_exact(tmc, orc, torch):
    heads, d, p, seq = 4, 32, 4, 3
    cap = 16
    table = np.array([2, 0, 3, 1], np.int32)
    pool = orc.f16(normal(307, (4 * heads * p * d,)))
    new = orc.f16(normal(308, (1, seq * heads * d)))
    pool_d = dev_f16(pool)
    valid = torch.tensor([7], dtype=torch.int32, device="cuda")
    tmc.paged_kv_append(dev_f16(new), valid, dev(table), pool_d, 1, seq, heads, d, cap, p, False)
    torch.cuda.synchronize()
    expect = orc.append_paged(new, pool, 1, heads, d, seq, cap, p, False, 7, table)
    assert np.array_equal(bits(pool_d), expect)
    # serving layout [page][heads][page][D], 3 active of 4 rows, one invalid
    max_b, max_pages = 4, cap // p
    tables = np.array([[5, 1, -1, -1], [0, 2, 7, -1], [3, -1, -1, -1], [6, 4, -1, -1]], np.int32)
    lengths = np.array([6, 9, 0, 8], np.int32)
    pool2 = orc.f16(normal(309, (8 * heads * p * d,)))
    new2 = orc.f16(normal(310, (max_b, heads * d)))
    pool2_d = dev_f16(pool2)
    active = torch.tensor([3], dtype=torch.int32, device="cuda")
    tmc.serving_kv_append(dev_f16(new2), dev(lengths), dev(tables), active, pool2_d, max_b, heads,
                          d, cap, p, True)
    torch.cuda.synchronize()
    expect2 = orc.append_serving(new2, pool2, max_b, heads, d, cap, p, True, lengths, tables, 3)
    assert np.array_equal(bits(pool2_d), expect2)


# ---------------------------------------------------------------- attention
def _ws(tmc, torch, batch, qh, kvh, d, cap):
    n = tmc.attention_workspace_bytes(batch, qh, kvh, d, cap)
    # per-split partial results (weighted sums, maxima, denominators); the
    # merge reads only the slots the split blocks wrote in this launch
    return torch.zeros(max(n // 4, 1), dtype=torch.float32, device="cuda") if n else None


@pytest.mark.parametrize("length", [128, 1024, 4095])
def test_c3_contiguous_decode_attention(tmc, orc, torch, length):
    heads, d, cap = 32, 128, 4096
    k = orc.f16(normal(301, (1, heads, cap, d)))
    v = orc.f16(normal(302, (1, heads, cap, d)))
    q = orc.f16(normal(303, (1, heads * d)))
    nk = orc.f16(normal(304, (1, heads * d)))
    nv = orc.f16(normal(305, (1, heads * d)))
    k_d, v_d = dev_f16(k), dev_f16(v)
    valid = torch.tensor([length + 1], dtype=torch.int32, device="cuda")
    tmc.kv_append(dev_f16(nk), valid, k_d, 1, 1, heads, d, cap, False)
    tmc.kv_append(dev_f16(nv), valid, v_d, 1, 1, heads, d, cap, False)
    out = torch.full((1, heads * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.decode_attention(dev_f16(q), k_d, v_d, valid, out, 1, heads, heads, d, cap,
                         _ws(tmc, torch, 1, heads, heads, d, cap))
    torch.cuda.synchronize()
    kk = orc.append_contiguous(nk, k.ravel(), 1, heads, d, 1, cap, False, length + 1)
    vv = orc.append_contiguous(nv, v.ravel(), 1, heads, d, 1, cap, False, length + 1)
    ref = orc.decode_attention(q, kk, vv, F16, heads, heads, d, cap, length + 1)
    assert_f16_path(values(out), ref, what=f"contiguous attention L={length}")


@pytest.mark.parametrize("valid,d,qh,kvh", [(1, 128, 32, 32), (256, 128, 8, 2), (257, 128, 8, 8),
                                            (513, 64, 4, 1), (700, 16, 4, 4), (2049, 32, 8, 1)])
def test_decode_attention_edges(tmc, orc, torch, valid, d, qh, kvh):
    cap = 2304
    b = 2
    k = orc.f16(normal(311, (b, kvh, cap, d)))
    v = orc.f16(normal(312, (b, kvh, cap, d)))
    q = orc.f16(normal(313, (b, qh * d)) * 2)
    out = torch.full((b, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    vl = torch.tensor([valid], dtype=torch.int32, device="cuda")
    tmc.decode_attention(dev_f16(q), dev_f16(k), dev_f16(v), vl, out, b, qh, kvh, d, cap,
                         _ws(tmc, torch, b, qh, kvh, d, cap))
    torch.cuda.synchronize()
    ref = orc.decode_attention(q, k, v, F16, qh, kvh, d, cap, valid)
    assert_f16_path(values(out), ref, what=f"attention valid={valid} d={d} group={qh // kvh}")


@pytest.mark.parametrize("valid,qh,kvh", [(31, 32, 32), (33, 8, 2), (161, 32, 32), (512, 8, 8),
                                           (1500, 16, 4), (3000, 32, 32)])
def test_contiguous_splits_follow_the_length(tmc, orc, torch, valid, qh, kvh):
    """A contiguous cache cuts each row into the capacity's split count of
    its own length (32-position steps), not of the capacity: lengths on
    both sides of the step and split boundaries at capacity 4096, batch 2,
    against the oracle."""
    b, d, cap = 2, 128, 4096
    k = orc.f16(normal(331, (b, kvh, cap, d)))
    v = orc.f16(normal(332, (b, kvh, cap, d)))
    q = orc.f16(normal(333, (b, qh * d)) * 2)
    out = torch.full((b, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    vl = torch.tensor([valid], dtype=torch.int32, device="cuda")
    tmc.decode_attention(dev_f16(q), dev_f16(k), dev_f16(v), vl, out, b, qh, kvh, d, cap,
                         _ws(tmc, torch, b, qh, kvh, d, cap))
    torch.cuda.synchronize()
    ref = orc.decode_attention(q, k, v, F16, qh, kvh, d, cap, valid)
    assert_f16_path(values(out), ref, what=f"attention valid={valid} group={qh // kvh}")


@pytest.mark.parametrize("b,valid,qh,kvh,cap", [(1, 1, 32, 32, 1024), (1, 33, 32, 32, 1024),
                                                 (1, 700, 32, 32, 1024), (1, 1024, 32, 32, 1024),
                                                 (2, 999, 8, 4, 1000), (3, 129, 4, 2, 160),
                                                 (9, 500, 32, 32, 512)])
def test_decode_attention_one_wide_split(tmc, orc, torch, b, valid, qh, kvh, cap):
    """Capacity <= 1024 (head_dim 128, GQA group <= 2) runs one split per
    (request, kv head): 16-wave blocks up to 256 such rows, 4-wave blocks
    beyond (the last case, 288 rows); no workspace, no combine."""
    d = 128
    assert tmc.attention_workspace_bytes(b, qh, kvh, d, cap) == 0
    k = orc.f16(normal(321, (b, kvh, cap, d)))
    v = orc.f16(normal(322, (b, kvh, cap, d)))
    q = orc.f16(normal(323, (b, qh * d)) * 2)
    out = torch.full((b, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    vl = torch.tensor([valid], dtype=torch.int32, device="cuda")
    tmc.decode_attention(dev_f16(q), dev_f16(k), dev_f16(v), vl, out, b, qh, kvh, d, cap, None)
    torch.cuda.synchronize()
    ref = orc.decode_attention(q, k, v, F16, qh, kvh, d, cap, valid)
    assert_f16_path(values(out), ref, what=f"wide attention b={b} valid={valid} group={qh // kvh}")


def _c4_inputs(orc, torch, batch=16, qh=32, kvh=8, d=128, p=16, pages=8192, max_pages=256):
    # contexts U[64, 4095] so that the appended token keeps valid <= 4096
    lengths = np.random.default_rng(403).integers(64, 4096, size=batch).astype(np.int32)
    perm = np.random.default_rng(404).permutation(pages).astype(np.int32)
    tables = np.full((batch, max_pages), -1, np.int32)
    cursor = 0
    for i, length in enumerate(lengths):
        need = (int(length) + 1 + p - 1) // p  # room for the appended token
        tables[i, :need] = perm[cursor:cursor + need]
        cursor += need
    k_pool = orc.f16(normal(401, (pages, kvh, p, d)))
    v_pool = orc.f16(normal(402, (pages, kvh, p, d)))
    q = orc.f16(normal(405, (batch, qh * d)))
    return lengths, tables, k_pool, v_pool, q


def test_c4_paged_gqa_attention(tmc, orc, torch):
    batch, qh, kvh, d, p, pages, max_pages = 16, 32, 8, 128, 16, 8192, 256
    lengths, tables, k_pool, v_pool, q = _c4_inputs(orc, torch)
    nk = orc.f16(normal(406, (batch, kvh * d)))
    nv = orc.f16(normal(407, (batch, kvh * d)))
    k_d, v_d = dev_f16(k_pool), dev_f16(v_pool)
    tables_d = dev(tables)
    valid = lengths + 1
    valid_d = dev(valid)
    active = torch.tensor([batch], dtype=torch.int32, device="cuda")
    cap = max_pages * p
    tmc.serving_kv_append(dev_f16(nk), valid_d, tables_d, active, k_d, batch, kvh, d, cap, p, True)
    tmc.serving_kv_append(dev_f16(nv), valid_d, tables_d, active, v_d, batch, kvh, d, cap, p, True)
    out = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.paged_decode_attention(dev_f16(q), k_d, v_d, valid_d, tables_d, active, out, batch, qh,
                               kvh, d, p, max_pages, kvh * p * d, p * d,
                               _ws(tmc, torch, batch, qh, kvh, d, cap))
    torch.cuda.synchronize()
    kp = orc.append_serving(nk, k_pool.ravel(), batch, kvh, d, cap, p, True, valid, tables, batch)
    vp = orc.append_serving(nv, v_pool.ravel(), batch, kvh, d, cap, p, True, valid, tables, batch)
    assert np.array_equal(bits(k_d).ravel(), kp)
    ref, written = orc.paged_attention(q, kp, vp, F16, qh, kvh, d, p, kvh * p * d, p * d, tables,
                                       max_pages, valid, batch)
    assert written.all()
    assert_f16_path(values(out), ref, what="paged GQA attention (C4)")


def test_paged_attention_workspace_reused_across_shapes(tmc, orc, torch):
    """One zeroed workspace serves launches of different shapes in turn:
    the arrival counters sit in a fixed area at the workspace's start that no
    launch's partials overlap, and every launch leaves them at zero.  A small
    batch with 16 splits per row, a larger batch with more (request, kv head)
    rows, a head_dim 64 launch (partials merged by a second launch), then the
    first shape again, each against the oracle."""
    p = 16
    cases = [  # batch, q heads, kv heads, head_dim, max_pages
        (2, 8, 2, 128, 128),
        (16, 32, 8, 128, 128),
        (4, 8, 8, 64, 128),
        (2, 8, 2, 128, 128),
    ]
    need = max(tmc.attention_workspace_bytes(b, qh, kvh, d, mp * p) for b, qh, kvh, d, mp in cases)
    assert all(tmc.attention_workspace_bytes(b, qh, kvh, d, mp * p) > 0
               for b, qh, kvh, d, mp in cases), "every case should split its rows"
    ws = torch.zeros(need // 4, dtype=torch.float32, device="cuda")
    for i, (batch, qh, kvh, d, max_pages) in enumerate(cases):
        pages = batch * max_pages
        k_pool = orc.f16(normal(430 + i, (pages, kvh, p, d)))
        v_pool = orc.f16(normal(440 + i, (pages, kvh, p, d)))
        q = orc.f16(normal(450 + i, (batch, qh * d)))
        lengths = np.random.default_rng(460 + i).integers(1, max_pages * p + 1,
                                                           size=batch).astype(np.int32)
        tables = np.random.default_rng(470 + i).permutation(pages).astype(np.int32)
        tables = tables.reshape(batch, max_pages)
        out = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
        active = torch.tensor([batch], dtype=torch.int32, device="cuda")
        tmc.paged_decode_attention(dev_f16(q), dev_f16(k_pool), dev_f16(v_pool), dev(lengths),
                                   dev(tables), active, out, batch, qh, kvh, d, p, max_pages,
                                   kvh * p * d, p * d, ws)
        torch.cuda.synchronize()
        ref, written = orc.paged_attention(q, k_pool, v_pool, F16, qh, kvh, d, p, kvh * p * d,
                                           p * d, tables, max_pages, lengths, batch)
        assert written.all()
        assert_f16_path(values(out), ref, what=f"workspace reuse, case {i} (b={batch}, d={d})")


@pytest.mark.parametrize("d,p,qh,max_pages", [(64, 16, 8, 8), (128, 16, 8, 8), (128, 8, 8, 8),
                                               (128, 16, 4, 32), (128, 8, 4, 32)])
def test_paged_attention_inactive_and_bad_pages_untouched(tmc, orc, torch, d, p, qh, max_pages):
    """Rows past the active count, rows whose range needs a missing page (a
    negative entry, or a page id past the pool) keep their output.  GQA group
    2 at max_pages 32 runs the one-split 16-wave blocks."""
    batch, kvh = 5, 2
    pages = 32
    k_pool = orc.f16(normal(410, (pages, kvh, p, d)))
    v_pool = orc.f16(normal(411, (pages, kvh, p, d)))
    q = orc.f16(normal(412, (batch, qh * d)))
    tables = np.full((batch, max_pages), -1, np.int32)
    tables[0, :3] = [4, 9, 1]
    tables[1, :2] = [7, -1]  # hole inside the valid range
    tables[2, :8] = np.arange(10, 18)
    tables[3, :1] = [pages + 3]  # past the end of the pool
    tables[4, :1] = [3]
    lengths = np.array([3 * p - 8, p + 4, 8 * p, 5, 5], np.int32)
    out = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    active = torch.tensor([4], dtype=torch.int32, device="cuda")
    cap = max_pages * p
    tmc.paged_decode_attention(dev_f16(q), dev_f16(k_pool), dev_f16(v_pool), dev(lengths),
                               dev(tables), active, out, batch, qh, kvh, d, p, max_pages,
                               kvh * p * d, p * d, _ws(tmc, torch, batch, qh, kvh, d, cap))
    torch.cuda.synchronize()
    got = values(out)
    oracle_tables = tables.copy()
    oracle_tables[3] = -1  # the oracle reads pools directly: give it the missing-page form
    ref, written = orc.paged_attention(q, k_pool, v_pool, F16, qh, kvh, d, p, kvh * p * d, p * d,
                                       oracle_tables, max_pages, lengths, 4)
    assert list(written.all(axis=1)) == [True, False, True, False, False]
    for row in (1, 3, 4):
        assert np.isnan(got[row]).all(), row
    assert_f16_path(got[[0, 2]], ref[[0, 2]], what="paged attention written rows")


@pytest.mark.parametrize("batch,qh,kvh,d,active", [(20, 32, 32, 128, 20), (20, 32, 16, 128, 17),
                                                   (16, 32, 8, 128, 16), (16, 32, 4, 128, 11),
                                                   (5, 8, 2, 64, 4)])
def test_paged_attention_packed_output_bit_exact(tmc, torch, batch, qh, kvh, d, active):
    """The packed output layout holds the row-major result's bits, unpacked
    by the activation packer (split merges in the kernel for GQA groups 1, 2
    and 4 at head_dim 128, the combine kernel for group 8 and at head_dim
    64); rows past the
    active count stay untouched in both layouts; two 16-row passes at
    batch 20."""
    p, max_pages, pages = 16, 64, 256
    rng = np.random.default_rng(420 + batch + kvh)
    lengths = rng.integers(1, max_pages * p + 1, size=batch).astype(np.int32)
    tables = rng.integers(0, pages, size=(batch, max_pages)).astype(np.int32)
    k_pool = torch.from_numpy(normal(421, (pages, kvh, p, d))).half().cuda()
    v_pool = torch.from_numpy(normal(422, (pages, kvh, p, d))).half().cuda()
    q = torch.from_numpy(normal(423, (batch, qh * d))).half().cuda()
    act = torch.tensor([active], dtype=torch.int32, device="cuda")
    args = (q, k_pool, v_pool, dev(lengths), dev(tables), act)
    shape = (batch, qh, kvh, d, p, max_pages, kvh * p * d, p * d)
    ws = _ws(tmc, torch, batch, qh, kvh, d, max_pages * p)
    rm = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.paged_decode_attention(*args, rm, *shape, ws)
    packed = tmc.pack_activations(torch.full_like(rm, float("nan")))
    tmc.paged_decode_attention(*args, packed, *shape, ws, layout=tmc.Y_PACKED)
    back = torch.empty_like(rm)
    tmc.pack_activations(packed, out=back, unpack=True, rows=batch, cols=qh * d)
    torch.cuda.synchronize()
    assert torch.equal(back.view(torch.int16), rm.view(torch.int16))
    assert not torch.isnan(rm[:active]).any() and torch.isnan(rm[active:]).all()
    with pytest.raises(RuntimeError, match="out_layout must be row_major or packed"):
        tmc.Runtime().resolve("paged_attention?max_batch=4&q_heads=8&head_dim=128&page_size=16"
                              "&max_pages=16&out_layout=tiled")


# ---------------------------------------------------------------- rope / embedding / argmax
def test_rope_decoder_and_serving(tmc, orc, torch):
    heads, d, cap, seq, batch = 4, 16, 32, 3, 2
    pairs = d // 2
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos, sin = np.cos(pos * freq).astype(np.float32), np.sin(pos * freq).astype(np.float32)
    x = orc.f16(normal(501, (batch, seq, heads * d)))
    out = torch.empty((batch, heads, seq, d), dtype=torch.float16, device="cuda")
    valid = 9
    tmc.rope(dev_f16(x), dev(cos), dev(sin), torch.tensor([valid], dtype=torch.int32,
                                                          device="cuda"),
             out, batch, seq, heads, d, cap)
    torch.cuda.synchronize()
    positions = np.tile(np.arange(valid - seq, valid), batch)
    ref = orc.rope(x.reshape(batch * seq, heads * d), cos, sin, F16, heads, d, positions)
    ref = ref.reshape(batch, seq, heads, d).transpose(0, 2, 1, 3)
    assert_f16_path(values(out), ref, what="decoder rope")
    assert pairs == cos.shape[1]
    # serving: one token per request at valid-1, inactive rows untouched
    xs = orc.f16(normal(502, (4, heads * d)))
    lengths = np.array([1, 30, 7, 5], np.int32)
    outs = torch.full((4, heads * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.serving_rope(dev_f16(xs), dev(cos), dev(sin), dev(lengths),
                     torch.tensor([3], dtype=torch.int32, device="cuda"), outs, 4, heads, d, cap)
    torch.cuda.synchronize()
    refs = orc.rope(xs, cos, sin, F16, heads, d, lengths - 1)
    got = values(outs)
    assert_f16_path(got[:3], refs[:3], what="serving rope")
    assert np.isnan(got[3]).all()


@pytest.mark.parametrize("qh,kvh,d", [(32, 32, 128), (32, 8, 128), (4, 2, 64), (2, 1, 12)])
def test_decode_rope_append_is_rope_then_append(tmc, orc, torch, qh, kvh, d):
    """Fused RoPE(q, k) + paged append of k, v (one fused projection row per
    request) equals tmc_serving_rope followed by tmc_serving_kv_append bit for
    bit, and the oracle's RoPE within the fp16-path tolerance; pages of other
    rows, rows at or past the active count and positions without a page stay
    untouched."""
    cap, p, batch = 64, 16, 5
    max_pages = cap // p
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos, sin = np.cos(pos * freq).astype(np.float32), np.sin(pos * freq).astype(np.float32)
    width = (qh + 2 * kvh) * d
    qkv = orc.f16(normal(511, (batch, width)))
    lengths = np.array([1, 17, 64, 33, 9], np.int32)
    pages = 24
    perm = np.random.default_rng(512).permutation(pages).astype(np.int32)
    tables = perm[:batch * max_pages].reshape(batch, max_pages).copy()
    tables[3, 2] = -1  # row 3's new token (position 32) has no page
    active = 4          # row 4 is padding
    pool0 = orc.f16(normal(513, (pages, kvh, p, d)))
    kp, vp = dev_f16(pool0), dev_f16(pool0.copy())
    q_out = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    args = (dev(cos), dev(sin), dev(lengths), dev(tables),
            torch.tensor([active], dtype=torch.int32, device="cuda"))
    tmc.decode_rope_append(dev_f16(qkv), *args, q_out, kp, vp, batch, qh, kvh, d, cap, p,
                           max_pages)
    # unfused path on the same inputs
    q_in = dev_f16(np.ascontiguousarray(qkv[:, :qh * d]))
    k_in = dev_f16(np.ascontiguousarray(qkv[:, qh * d:(qh + kvh) * d]))
    v_in = dev_f16(np.ascontiguousarray(qkv[:, (qh + kvh) * d:]))
    q_ref = torch.full_like(q_out, float("nan"))
    k_rot = torch.empty((batch, kvh * d), dtype=torch.float16, device="cuda")
    tmc.serving_rope(q_in, dev(cos), dev(sin), dev(lengths), args[4], q_ref, batch, qh, d, cap)
    tmc.serving_rope(k_in, dev(cos), dev(sin), dev(lengths), args[4], k_rot, batch, kvh, d, cap)
    kp2, vp2 = dev_f16(pool0), dev_f16(pool0.copy())
    tmc.serving_kv_append(k_rot, dev(lengths), dev(tables), args[4], kp2, batch, kvh, d, cap, p,
                          False)
    tmc.serving_kv_append(v_in, dev(lengths), dev(tables), args[4], vp2, batch, kvh, d, cap, p,
                          False)
    torch.cuda.synchronize()
    assert np.array_equal(bits(q_out)[:active], bits(q_ref)[:active])
    assert np.isnan(values(q_out)[active:]).all()
    assert np.array_equal(bits(kp), bits(kp2)) and np.array_equal(bits(vp), bits(vp2))
    # oracle: rotation within tolerance, value append bit-exact
    ref_q = orc.rope(qkv[:active, :qh * d], cos, sin, F16, qh, d, lengths[:active] - 1)
    assert_f16_path(values(q_out)[:active], ref_q, what="fused rope q")
    ref_v = orc.append_serving(np.ascontiguousarray(qkv[:, (qh + kvh) * d:]), pool0.ravel(), batch,
                               kvh, d, cap, p, False, lengths, tables, active)
    assert np.array_equal(bits(vp).ravel(), ref_v)
    changed = np.flatnonzero((bits(kp) != pool0).reshape(pages, -1).any(axis=1))
    expect = {int(tables[b, (lengths[b] - 1) // p]) for b in range(active)} - {-1}
    assert set(changed.tolist()) <= expect


QKV_ROPE_CONFIGS = [(1, 2, u, ks) for u in (2, 4) for ks in (1, 2, 4)]


@pytest.mark.parametrize("qh,kvh,d,hidden", [(32, 32, 128, 4096), (32, 8, 128, 1024),
                                             (4, 2, 64, 264), (2, 1, 12, 24)])
def test_qkv_rope_append_equals_gemv_then_rope_append(tmc, orc, torch, qh, kvh, d, hidden):
    """The batch-1 q.k.v projection with RoPE and the paged append in its
    epilogue writes the bits of tmc_gemv_f16_config (same k split) followed by
    tmc_decode_rope_append, for every dot configuration with two rows per
    wave; the skip rules (inactive request, length outside [1, capacity],
    missing page) leave q and both pools untouched."""
    cap, p = 64, 16
    max_pages = cap // p
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos, sin = np.cos(pos * freq).astype(np.float32), np.sin(pos * freq).astype(np.float32)
    width = (qh + 2 * kvh) * d
    x = dev_f16(orc.f16(normal(531, (1, hidden))))
    w = dev_f16(orc.f16(normal(532, (width, hidden)) * 0.05))
    pages = 12
    pool0 = orc.f16(normal(533, (pages, kvh, p, d)))
    table = np.array([7, 2, -1, 5], np.int32)
    cos_d, sin_d, table_d = dev(cos), dev(sin), dev(table)
    one = torch.tensor([1], dtype=torch.int32, device="cuda")
    cases = [(20, 1), (1, 1), (64, 1), (40, 1), (20, 0), (0, 1), (65, 1)]  # (valid, active)
    for cfg in QKV_ROPE_CONFIGS:
        for valid, active in cases:
            lengths = torch.tensor([valid], dtype=torch.int32, device="cuda")
            act = torch.tensor([active], dtype=torch.int32, device="cuda")
            kp, vp = dev_f16(pool0), dev_f16(pool0.copy())
            q = torch.full((1, qh * d), float("nan"), dtype=torch.float16, device="cuda")
            tmc.qkv_rope_append(x, w, cos_d, sin_d, lengths, table_d, act, q, kp, vp, qh, kvh, d,
                                cap, p, config=cfg)
            qkv = torch.empty((1, width), dtype=torch.float16, device="cuda")
            tmc.gemv_config(x, w, qkv, tmc.GemvConfig(1, 1, cfg[2], cfg[3]))
            kp2, vp2 = dev_f16(pool0), dev_f16(pool0.copy())
            q2 = torch.full_like(q, float("nan"))
            tmc.decode_rope_append(qkv, cos_d, sin_d, lengths, table_d, act, q2, kp2, vp2, 1, qh,
                                   kvh, d, cap, p, max_pages)
            torch.cuda.synchronize()
            what = f"config {cfg} valid {valid} active {active}"
            assert np.array_equal(bits(q), bits(q2)), what
            assert np.array_equal(bits(kp), bits(kp2)), what
            assert np.array_equal(bits(vp), bits(vp2)), what
            wrote = active == 1 and 1 <= valid <= cap and table[(valid - 1) // p] >= 0
            assert (not np.array_equal(bits(kp), pool0)) == wrote, what
            assert np.isnan(values(q)).all() == (active != 1 or not 1 <= valid <= cap), what
    with pytest.raises(tmc.TmcError, match="rows_per_wave 2"):
        tmc.qkv_rope_append(x, w, cos_d, sin_d, one, table_d, one, q, kp, vp, qh, kvh, d, cap, p,
                            config=(1, 1, 4, 4))


@pytest.mark.parametrize("batch,layout,cfg_t", [(2, 0, None), (5, 1, None), (16, 1, (3, 1, 1, 4)),
                                                (17, 1, (3, 1, 4, 1)), (16, 0, (3, 1, 2, 8))])
def test_qkv_rope_append_packed_equals_gemm_then_rope_append(tmc, orc, torch, batch, layout,
                                                             cfg_t):
    """The batched q.k.v projection over packed weights with RoPE and the
    paged append in its epilogue writes the bits of tmc_gemm_packed_ex_f16
    (same configuration and x layout) followed by tmc_decode_rope_append:
    every request's own length and block table, rows past the active count,
    lengths outside [1, capacity] and missing pages skipped."""
    qh, kvh, d, hidden, cap, p = 8, 4, 64, 512, 64, 16
    mp = cap // p
    cfg = tmc.GemvConfig(*cfg_t) if cfg_t else None
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos = dev(np.cos(pos * freq).astype(np.float32))
    sin = dev(np.sin(pos * freq).astype(np.float32))
    width = (qh + 2 * kvh) * d
    xr = orc.f16(normal(551, (batch, hidden)))
    w = dev_f16(orc.f16(normal(552, (width, hidden), 0.05)))
    packed = tmc.pack_weights(w)
    x_rm = dev_f16(xr)
    x = tmc.pack_activations(x_rm) if layout else x_rm
    rng = np.random.default_rng(553)
    pages = batch * mp + 4
    tables = rng.permutation(pages)[:batch * mp].astype(np.int32).reshape(batch, mp)
    lengths = rng.integers(1, cap + 1, batch).astype(np.int32)
    lengths[0] = 0            # outside [1, capacity]
    lengths[-1] = cap + 1
    if batch > 2:
        lengths[1] = 20
        tables[1, 1] = -1     # missing page for row 1's token
    active = batch - 1 if batch > 2 else batch
    pool0 = orc.f16(normal(554, (pages, kvh, p, d)))
    args = (cos, sin, dev(lengths), dev(tables), torch.tensor([active], dtype=torch.int32,
                                                               device="cuda"))
    kp, vp = dev_f16(pool0), dev_f16(pool0.copy())
    q = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.qkv_rope_append_packed(x, packed, *args, q, kp, vp, batch, hidden, qh, kvh, d, cap, p, mp,
                               layout, cfg)
    qkv = torch.empty((batch, width), dtype=torch.float16, device="cuda")
    tmc.gemm_packed_ex(x, packed, qkv, batch, hidden, width, layout, cfg)
    kp2, vp2 = dev_f16(pool0), dev_f16(pool0.copy())
    q2 = torch.full_like(q, float("nan"))
    tmc.decode_rope_append(qkv, *args, q2, kp2, vp2, batch, qh, kvh, d, cap, p, mp)
    torch.cuda.synchronize()
    assert np.array_equal(bits(q), bits(q2))
    assert np.array_equal(bits(kp), bits(kp2)) and np.array_equal(bits(vp), bits(vp2))
    assert np.isnan(values(q)[0]).all()
    if batch > 2:
        assert not np.isnan(values(q)[2]).all()


@pytest.mark.parametrize("cfg_t", [(1, 2, 2, 4), (1, 2, 4, 4), None])
def test_norm_qkv_rope_append_equals_norm_then_fused_projection(tmc, orc, torch, cfg_t):
    """The Add+RMSNorm (or RMSNorm) prologue in the q.k.v RoPE append kernel
    reproduces tmc_add_rmsnorm (tmc_rmsnorm; one chunk per thread at hidden
    1024) followed by tmc_qkv_rope_append_f16 with the same configuration bit
    for bit, residual sum included."""
    qh, kvh, d, hidden, cap, p = 32, 16, 128, 1024, 64, 16
    cfg = tmc.GemvConfig(*cfg_t) if cfg_t else None
    ref_cfg = cfg_t or (1, 2, 4, 4)
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos = dev(np.cos(pos * freq).astype(np.float32))
    sin = dev(np.sin(pos * freq).astype(np.float32))
    width = (qh + 2 * kvh) * d
    h = dev_f16(orc.f16(normal(541, (1, hidden))))
    r = dev_f16(orc.f16(normal(542, (1, hidden))))
    gamma = dev_f16(orc.f16(uniform(543, (hidden,), 0.5, 1.5)))
    w = dev_f16(orc.f16(normal(544, (width, hidden), 0.05)))
    pool0 = orc.f16(normal(545, (8, kvh, p, d)))
    table = dev(np.array([3, 6, 1, 4], np.int32))
    lengths = torch.tensor([37], dtype=torch.int32, device="cuda")
    one = torch.tensor([1], dtype=torch.int32, device="cuda")
    for add in (True, False):
        s_ref = torch.empty((1, hidden), dtype=torch.float16, device="cuda")
        n_ref = torch.empty_like(s_ref)
        if add:
            tmc.add_rmsnorm(r, h, gamma, s_ref, n_ref, 1e-6)
        else:
            tmc.rmsnorm(r, gamma, n_ref, 1e-6)
        kp_ref, vp_ref = dev_f16(pool0), dev_f16(pool0.copy())
        q_ref = torch.full((1, qh * d), float("nan"), dtype=torch.float16, device="cuda")
        tmc.qkv_rope_append(n_ref, w, cos, sin, lengths, table, one, q_ref, kp_ref, vp_ref, qh,
                            kvh, d, cap, p, config=ref_cfg)
        kp, vp = dev_f16(pool0), dev_f16(pool0.copy())
        q = torch.full_like(q_ref, float("nan"))
        s_out = torch.full((1, hidden), 7.0, dtype=torch.float16, device="cuda")
        tmc.add_rmsnorm_qkv_rope_append(r, h if add else None, gamma, w, s_out if add else None,
                                        cos, sin, lengths, table, one, q, kp, vp, qh, kvh, d, cap,
                                        p, 1e-6, config=cfg)
        torch.cuda.synchronize()
        what = f"cfg {cfg_t} add={add}"
        assert np.array_equal(bits(q), bits(q_ref)), what
        assert np.array_equal(bits(kp), bits(kp_ref)), what
        assert np.array_equal(bits(vp), bits(vp_ref)), what
        assert not np.array_equal(bits(kp), pool0), what
        if add:
            assert np.array_equal(bits(s_out), bits(s_ref)), what
        else:
            assert torch.all(s_out == 7.0)


def test_embedding_and_argmax(tmc, orc, torch):
    vocab, hidden = 1000, 64
    table = orc.f16(normal(601, (vocab, hidden)))
    tokens = np.array([5, 999, -1, 1000, 0], np.int32)
    out = torch.full((5, hidden), float("nan"), dtype=torch.float16, device="cuda")
    tmc.embedding(dev(tokens), dev_f16(table), out)
    torch.cuda.synchronize()
    got = bits(out)
    assert np.array_equal(got[[0, 1, 4]], table[[5, 999, 0]])
    assert np.isnan(values(out)[[2, 3]]).all()
    logits = normal(602, (4, 32000))
    logits[1, 100] = logits[1, 31999] = 50.0  # tie -> lowest index
    logits[2, :] = -np.inf
    logits[3, 7] = np.nan
    toks = torch.empty(4, dtype=torch.int32, device="cuda")
    tmc.argmax(dev(logits), toks)
    torch.cuda.synchronize()
    assert list(toks.cpu().numpy()) == list(orc.argmax(logits))
    assert toks.cpu().numpy()[1] == 100 and toks.cpu().numpy()[2] == 0


@pytest.mark.parametrize("rows,vocab", [(16, 32000), (3, 32001), (2, 4099), (1, 5), (2, 40000)])
def test_argmax_ties_nan_and_tails(tmc, orc, torch, rows, vocab):
    """Vector (vocab % 4 == 0) and scalar paths, ties across threads and
    load rounds, NaN entries, an all -inf row, the last element."""
    logits = normal(603 + vocab, (rows, vocab))
    logits[0, vocab - 1] = 60.0
    if rows > 1:
        logits[1, :] = -np.inf
        logits[1, vocab // 2] = np.nan
    if rows > 2:
        logits[2, 3] = logits[2, vocab - 2] = logits[2, 1024 * 4 + 1] = 70.0  # tie -> 3
    toks = torch.empty(rows, dtype=torch.int32, device="cuda")
    tmc.argmax(dev(logits), toks)
    torch.cuda.synchronize()
    got = list(toks.cpu().numpy())
    assert got == list(orc.argmax(logits))
    assert got[0] == vocab - 1
    if rows > 1:
        assert got[1] == 0
    if rows > 2:
        assert got[2] == 3


def test_read_probe_reads_without_writing(tmc, torch):
    """tmc_read_probe reads every byte and writes only its sink, and only when
    a block sum equals 1234.5: zeros and N(0, 1) data leave the sink alone;
    sizes that are not a multiple of 16 are refused."""
    src = torch.zeros(1 << 20, dtype=torch.float32, device="cuda")
    sink = torch.full((2,), 7.0, device="cuda")
    tmc.read_probe(src, src.numel() * 4, sink)
    src.normal_()
    tmc.read_probe(src, src.numel() * 4 - 48, sink)
    torch.cuda.synchronize()
    assert sink.tolist() == [7.0, 7.0]
    with pytest.raises(RuntimeError, match="multiple of 16"):
        tmc.read_probe(src, 40, sink)


def test_fill_normal_statistics(tmc, torch):
    t = torch.empty(1 << 20, dtype=torch.float16, device="cuda")
    tmc.fill_normal(t, 77, 0.0, 0.02)
    u = torch.empty(1 << 20, dtype=torch.float16, device="cuda")
    tmc.fill_normal(u, 77, 0.0, 0.02)
    torch.cuda.synchronize()
    a = values(t)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 2e-4
    assert np.array_equal(bits(t), bits(u))  # deterministic in the seed


CONFIGS = ([(1, r, u, k) for r in (1, 2) for u in (2, 4) for k in (1, 2, 4)] +
           [(2, nt, u, ks) for nt in (1, 2) for u in (1, 2) for ks in (1, 2, 4, 8, 16)
            if nt * ks <= 16] +
           # MFMA row tiles: the gated pair doubles the LDS partials, so
           # tiles * k_split <= 32 keeps both within 64 KiB
           [(3, rt, u, ks) for rt in (1, 2, 4) for u in (1, 2, 4) for ks in (1, 2, 4, 8, 16)
            if rt * ks <= 32 and not (u == 4 and rt == 4)] +
           [(4, 1, 1, 1)])


@pytest.mark.parametrize("algo,rpw,unroll,ks", CONFIGS)
def test_gemv_and_gated_mlp_every_config(tmc, orc, torch, algo, rpw, unroll, ks):
    """Every tuner candidate is parity-checked, at a shape with K and N tails."""
    cfg = tmc.GemvConfig()
    cfg.algorithm, cfg.rows_per_wave, cfg.unroll, cfg.k_split = algo, rpw, unroll, ks
    for batch in ((1, 3, 8) if algo == 1 else (1, 5, 16, 20)):
        # 9.06 K tiles of 128, 145 16-byte chunks, N tail of 8 (the linear
        # baseline also takes a K that is not a multiple of 8)
        k, n = (1160, 200) if algo != 4 else (1163, 200)
        x = orc.f16(normal(220 + batch, (batch, k)))
        w = orc.f16(normal(221, (n, k), 0.02))
        w2 = orc.f16(normal(222, (n, k), 0.02))
        y = torch.empty((batch, n), dtype=torch.float32, device="cuda")
        tmc.gemv_config(dev_f16(x), dev_f16(w), y, cfg)
        g = torch.empty((batch, n), dtype=torch.float16, device="cuda")
        tmc.gate_up_silu_config(dev_f16(x), dev_f16(w), dev_f16(w2), g, cfg)
        torch.cuda.synchronize()
        assert_f32_rel(values(y), orc.linear(x, w, F16), what=f"cfg {cfg.astuple()} b{batch}")
        assert_f16_path(values(g), orc.gated_mlp(x, w, w2, F16),
                        what=f"gated cfg {cfg.astuple()} b{batch}")


# ---------------------------------------------------------------- packed weights
def _pack_reference(w_bits):
    """Numpy restatement of the packed layout (include/tmc_hip.h): tile
    (n // 16, k // 32), lane n % 16 + 16 * ((k % 32) // 8), element k % 8."""
    n, k = w_bits.shape
    nt, kc = (n + 15) // 16, (k + 31) // 32
    padded = np.zeros((nt * 16, kc * 32), np.uint16)
    padded[:n, :k] = w_bits
    # [nt, 16 rows, kc, 4 groups, 8] -> [nt, kc, 4 groups, 16 rows, 8]
    t = padded.reshape(nt, 16, kc, 4, 8).transpose(0, 2, 3, 1, 4)
    return t.reshape(-1)


@pytest.mark.parametrize("n,k", [(16, 32), (200, 1160), (33, 8), (4096, 4096)])
def test_pack_weights_layout_bit_exact(tmc, orc, torch, n, k):
    w = orc.f16(normal(340, (n, k)))
    packed = tmc.pack_weights(dev_f16(w))
    torch.cuda.synchronize()
    assert packed.numel() == tmc.packed_weight_elements(n, k)
    assert np.array_equal(bits(packed), _pack_reference(w))


PACKED_CONFIGS = [(u, ks) for u in (1, 2, 4) for ks in (1, 2, 4, 8, 16)]


@pytest.mark.parametrize("unroll,ks", PACKED_CONFIGS)
def test_packed_gemm_and_gated_every_config(tmc, orc, torch, unroll, ks):
    cfg = tmc.GemvConfig(3, 1, unroll, ks)
    for batch, k, n in ((2, 1160, 200), (16, 1160, 200), (20, 4096, 48), (5, 8, 40)):
        x = orc.f16(normal(350 + batch, (batch, k)))
        w = orc.f16(normal(351, (n, k), 0.02))
        w2 = orc.f16(normal(352, (n, k), 0.02))
        pw, pw2 = tmc.pack_weights(dev_f16(w)), tmc.pack_weights(dev_f16(w2))
        y = torch.empty((batch, n), dtype=torch.float32, device="cuda")
        tmc.gemm_packed(dev_f16(x), pw, y, n, cfg)
        g = torch.empty((batch, n), dtype=torch.float16, device="cuda")
        tmc.gate_up_silu_packed(dev_f16(x), pw, pw2, g, n, cfg)
        torch.cuda.synchronize()
        what = f"packed u{unroll} ks{ks} b{batch} k{k} n{n}"
        assert_f32_rel(values(y), orc.linear(x, w, F16), what=what)
        assert_f16_path(values(g), orc.gated_mlp(x, w, w2, F16), what="gated " + what)


@pytest.mark.parametrize("batch,k,n,out_dtype", [
    (16, 4096, 12288, F16), (16, 4096, 4096, F32), (8, 11008, 4096, F16), (16, 4096, 32000, F32),
    (33, 256, 72, F32), (1, 4096, 256, F16),
])
def test_packed_gemm_default_configs(tmc, orc, torch, batch, k, n, out_dtype):
    x = orc.f16(normal(360, (batch, k)))
    w = orc.f16(normal(361, (n, k), 0.02))
    y = torch.empty((batch, n), dtype=torch.float32 if out_dtype == F32 else torch.float16,
                    device="cuda")
    tmc.gemm_packed(dev_f16(x), tmc.pack_weights(dev_f16(w)), y, n)
    torch.cuda.synchronize()
    ref = orc.linear(x, w, F16)
    if out_dtype == F32:
        assert_f32_rel(values(y), ref, what=f"packed default b{batch} n{n}")
    else:
        assert_f16_path(values(y), ref, what=f"packed default b{batch} n{n}")


def test_packed_gemm_rejects_bad_arguments(tmc, torch):
    x = torch.zeros((2, 12), dtype=torch.float16, device="cuda")
    p = torch.zeros(4096, dtype=torch.float16, device="cuda")
    y = torch.zeros((2, 16), dtype=torch.float32, device="cuda")
    with pytest.raises(tmc.TmcError):
        tmc.gemm_packed(x, p, y, 16)                            # in_features % 8 != 0
    with pytest.raises(tmc.TmcError):
        tmc.gemm_packed(x[:, :8].contiguous(), p, y, 16, tmc.GemvConfig(3, 1, 3, 4))  # unroll 3


# ---------------------------------------------------------------- fused norm + GEMV
DOT_CONFIGS = [(1, r, u, k) for r in (1, 2) for u in (2, 4) for k in (1, 2, 4)]


def _one_chunk_norm_threads(k):
    """A norm thread count with at most one 16-byte chunk per thread."""
    t = 256
    while t * 8 < k:
        t *= 2
    return t


@pytest.mark.parametrize("cfg_t", [(1, 1, 2, 4), (1, 2, 4, 4), None])
def test_fused_norm_gemv_equals_two_kernels_bit_exact(tmc, orc, torch, cfg_t):
    """The batch-1 GEMV / gated MLP with Add+RMSNorm (or RMSNorm) folded in
    reproduces tmc_add_rmsnorm_threads (tmc_rmsnorm_threads) with one chunk
    per thread followed by the dot GEMV at k split 4 bit for bit, residual
    sum included; rows_per_wave 1 or 2 rows per block, odd row counts."""
    cfg = tmc.GemvConfig(*cfg_t) if cfg_t else None
    for k, n in ((4096, 201), (1160, 4096), (1024, 9000), (8192, 300), (64, 3)):
        threads = _one_chunk_norm_threads(k)
        h = dev_f16(orc.f16(normal(370, (1, k))))
        r = dev_f16(orc.f16(normal(371, (1, k))))
        gamma = dev_f16(orc.f16(uniform(372, (k,), 0.5, 1.5)))
        w = dev_f16(orc.f16(normal(373, (n, k), 0.02)))
        w2 = dev_f16(orc.f16(normal(374, (n, k), 0.02)))
        ref_cfg = ref_gated = tmc.GemvConfig(1, 1, 2, 4)  # the k split fixes the order
        for add in (True, False):
            s_ref = torch.empty((1, k), dtype=torch.float16, device="cuda")
            n_ref = torch.empty_like(s_ref)
            if add:
                tmc.add_rmsnorm_threads(r, h, gamma, s_ref, n_ref, 1e-6, threads)
            else:
                tmc.rmsnorm_threads(r, gamma, n_ref, 1e-6, threads)
            y_ref = torch.empty((1, n), dtype=torch.float32, device="cuda")
            tmc.gemv_config(n_ref, w, y_ref, ref_cfg)
            g_ref = torch.empty((1, n), dtype=torch.float16, device="cuda")
            tmc.gate_up_silu_config(n_ref, w, w2, g_ref, ref_gated)
            s_out = torch.full((1, k), 7.0, dtype=torch.float16, device="cuda")
            y = torch.empty((1, n), dtype=torch.float32, device="cuda")
            tmc.add_rmsnorm_gemv(r, h if add else None, gamma, w, s_out if add else None, y, 1e-6,
                                 cfg)
            g = torch.empty((1, n), dtype=torch.float16, device="cuda")
            s2 = torch.empty((1, k), dtype=torch.float16, device="cuda")
            tmc.add_rmsnorm_gate_up_silu(r, h if add else None, gamma, w, w2, s2 if add else None,
                                         g, 1e-6, cfg)
            torch.cuda.synchronize()
            what = f"cfg {cfg_t} k{k} n{n} add={add}"
            assert torch.equal(y, y_ref), what
            assert np.array_equal(bits(g), bits(g_ref)), what
            if add:
                assert np.array_equal(bits(s_out), bits(s_ref)), what
                assert np.array_equal(bits(s2), bits(s_ref)), what
            else:
                assert torch.all(s_out == 7.0)


PERSISTENT_CONFIGS = [(5, 1, 1, 4), (5, 2, 1, 4)]


@pytest.mark.parametrize("cfg_t", PERSISTENT_CONFIGS)
def test_persistent_dot_equals_dot_bit_exact(tmc, orc, torch, cfg_t):
    """Algorithm 5 (the persistent batch-1 dot) sums each row in the order of
    the dot GEMV at k split 4: lane chunks in K order, then the four waves in
    order.  Shapes cover one to eight chunks per lane (K 64 .. 16384), row
    tails, grids that hold fewer groups than resident blocks and grids capped
    at 32 groups per block; fp16 and fp32 outputs; and the oracle."""
    cfg = tmc.GemvConfig(*cfg_t)
    dot = tmc.GemvConfig(1, 1, 2, 4)
    for k, n in ((4096, 4096), (11008, 4096), (4096, 11008), (1160, 200), (64, 9),
                 (12288, 77), (16384, 300), (1024, 70001)):
        x = orc.f16(normal(380, (1, k)))
        w = orc.f16(normal(381, (n, k), 0.02))
        for out_dtype in (torch.float16, torch.float32):
            y = torch.full((1, n), float("nan"), dtype=out_dtype, device="cuda")
            want = torch.empty_like(y)
            tmc.gemv_config(dev_f16(x), dev_f16(w), y, cfg)
            tmc.gemv_config(dev_f16(x), dev_f16(w), want, dot)
            torch.cuda.synchronize()
            what = f"cfg {cfg_t} k{k} n{n} {out_dtype}"
            assert torch.equal(y, want), what
            if out_dtype == torch.float32 and n * k <= 4096 * 11008:
                assert_f32_rel(values(y), orc.linear(x, w, F16), what=what)


def test_persistent_dot_rejects_unsupported_shapes(tmc, torch):
    """Batches above 1 and K above 16384 are refused, not run."""
    cfg = tmc.GemvConfig(5, 1, 1, 4)
    w = torch.zeros((8, 16392), dtype=torch.float16, device="cuda")
    x = torch.zeros((1, 16392), dtype=torch.float16, device="cuda")
    y = torch.zeros((1, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="persistent dot"):
        tmc.gemv_config(x, w, y, cfg)
    w2 = torch.zeros((8, 64), dtype=torch.float16, device="cuda")
    x2 = torch.zeros((2, 64), dtype=torch.float16, device="cuda")
    y2 = torch.zeros((2, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="persistent dot"):
        tmc.gemv_config(x2, w2, y2, cfg)
    with pytest.raises(RuntimeError, match="k_split 4"):
        tmc.gemv_config(x2[:1], w2, y2[:1], tmc.GemvConfig(5, 1, 1, 2))


@pytest.mark.parametrize("cfg_t", DOT_CONFIGS + PERSISTENT_CONFIGS + [None])
def test_gemv_residual_equals_gemv_then_add_bit_exact(tmc, orc, torch, cfg_t):
    """h(h(W x) + residual) in the GEMV epilogue (emitLinearResidual) against
    tmc_gemv_f16 with the same configuration followed by tmc_add, and against
    the oracle; the residual may be the output buffer's neighbour, not the
    output itself."""
    cfg = tmc.GemvConfig(*cfg_t) if cfg_t else None
    for k, n in ((4096, 4096), (11008, 4096), (1160, 200), (64, 9)):
        x = orc.f16(normal(390, (1, k)))
        w = orc.f16(normal(391, (n, k), 0.02))
        res = orc.f16(normal(392, (1, n)))
        y = torch.full((1, n), float("nan"), dtype=torch.float16, device="cuda")
        tmc.gemv_residual(dev_f16(x), dev_f16(w), dev_f16(res), y, cfg)
        proj = torch.empty((1, n), dtype=torch.float16, device="cuda")
        tmc.gemv_config(dev_f16(x), dev_f16(w), proj, cfg or tmc.default_config(1, k, n))
        want = torch.empty_like(proj)
        tmc.add(proj, dev_f16(res), want)
        torch.cuda.synchronize()
        what = f"cfg {cfg_t} k{k} n{n}"
        assert np.array_equal(bits(y), bits(want)), what
        if cfg_t is None:
            ref = orc.f16_values(res).astype(np.float64) + orc.store(orc.linear(x, w, F16), F16)
            assert_f16_path(values(y), ref, what=what)


def test_fused_norm_gemv_matches_oracle_and_rejects_batches(tmc, orc, torch):
    k, n = 4096, 11008
    h = orc.f16(normal(380, (1, k)))
    r = orc.f16(normal(381, (1, k)))
    gamma = orc.f16(uniform(382, (k,), 0.5, 1.5))
    wg = orc.f16(normal(383, (n, k), 0.02))
    wu = orc.f16(normal(384, (n, k), 0.02))
    s_out = torch.empty((1, k), dtype=torch.float16, device="cuda")
    g = torch.empty((1, n), dtype=torch.float16, device="cuda")
    tmc.add_rmsnorm_gate_up_silu(dev_f16(r), dev_f16(h), dev_f16(gamma), dev_f16(wg), dev_f16(wu),
                                 s_out, g, 1e-6)
    torch.cuda.synchronize()
    s_ref, n_ref = orc.add_rmsnorm(r, h, gamma, F16, 1e-6)
    assert_f16_path(values(s_out), s_ref, what="fused residual sum")
    n_chain = orc.f16(orc.store(n_ref, F16))
    assert_f16_path(values(g), orc.gated_mlp(n_chain, wg, wu, F16), what="fused gated mlp")
    x2 = torch.zeros((2, k), dtype=torch.float16, device="cuda")
    with pytest.raises(tmc.TmcError):
        tmc.add_rmsnorm_gemv(x2, x2, dev_f16(gamma), dev_f16(wg), x2,
                             torch.empty((2, n), dtype=torch.float32, device="cuda"), 1e-6)


# ---------------------------------------------------------------- packed activations
def _pack_act_reference(a_bits):
    """Fragment order of A [rows, cols] (include/tmc_hip.h), unwritten slots 0."""
    rows, cols = a_bits.shape
    passes, kc = (rows + 15) // 16, (cols + 31) // 32
    padded = np.zeros((passes * 16, kc * 32), np.uint16)
    padded[:rows, :cols] = a_bits
    return padded.reshape(passes, 16, kc, 4, 8).transpose(0, 2, 3, 1, 4).reshape(-1)


def _unwritten_mask(rows, cols):
    """Slots of the fragment order that hold real (row, col) elements."""
    passes, kc = (rows + 15) // 16, (cols + 31) // 32
    live = np.zeros((passes * 16, kc * 32), bool)
    live[:rows, :cols] = True
    return live.reshape(passes, 16, kc, 4, 8).transpose(0, 2, 3, 1, 4).reshape(-1)


@pytest.mark.parametrize("rows,cols", [(1, 8), (5, 40), (16, 4096), (20, 4096), (33, 1160)])
def test_pack_activations_layout_and_round_trip(tmc, orc, torch, rows, cols):
    a = orc.f16(normal(390, (rows, cols)))
    packed = tmc.pack_activations(dev_f16(a))
    back = torch.empty((rows, cols), dtype=torch.float16, device="cuda")
    tmc.pack_activations(packed, back, unpack=True, rows=rows, cols=cols)
    torch.cuda.synchronize()
    live = _unwritten_mask(rows, cols)
    assert packed.numel() == tmc.packed_activation_elements(rows, cols) == live.size
    assert np.array_equal(bits(packed)[live], _pack_act_reference(a)[live])
    assert np.array_equal(bits(back), a)


@pytest.mark.parametrize("rows", [1, 5, 16, 20])
def test_add_rmsnorm_packed_output_bit_exact(tmc, orc, torch, rows):
    k = 4096
    h = dev_f16(orc.f16(normal(391, (rows, k))))
    r = dev_f16(orc.f16(normal(392, (rows, k))))
    gamma = dev_f16(orc.f16(uniform(393, (k,), 0.5, 1.5)))
    s_ref, n_ref = torch.empty((rows, k), dtype=torch.float16, device="cuda"), None
    n_ref = torch.empty_like(s_ref)
    # width 4096 writes the packed rows with the 512-thread kernel
    tmc.add_rmsnorm_threads(r, h, gamma, s_ref, n_ref, 1e-6, 512)
    s_out = torch.empty_like(s_ref)
    n_packed = torch.empty(tmc.packed_activation_elements(rows, k), dtype=torch.float16,
                           device="cuda")
    tmc.add_rmsnorm_ex(r, h, gamma, s_out, n_packed, 1e-6, tmc.Y_PACKED)
    n_only = torch.empty_like(n_packed)
    tmc.add_rmsnorm_ex(r, None, gamma, None, n_only, 1e-6, tmc.Y_PACKED)
    plain = torch.empty_like(s_ref)
    tmc.rmsnorm_threads(r, gamma, plain, 1e-6, 512)
    torch.cuda.synchronize()
    live = _unwritten_mask(rows, k)
    assert np.array_equal(bits(s_out), bits(s_ref))
    assert np.array_equal(bits(n_packed)[live], _pack_act_reference(bits(n_ref))[live])
    assert np.array_equal(bits(n_only)[live], _pack_act_reference(bits(plain))[live])


@pytest.mark.parametrize("layout", [1, 2, 3])
def test_packed_gemm_activation_layouts_bit_exact(tmc, orc, torch, layout):
    """x packed and/or y packed gives the same bits as row-major activations."""
    for batch, k, n in ((5, 1160, 200), (16, 4096, 4096), (20, 4096, 11008)):
        x = dev_f16(orc.f16(normal(394 + batch, (batch, k))))
        w = dev_f16(orc.f16(normal(395, (n, k), 0.02)))
        w2 = dev_f16(orc.f16(normal(396, (n, k), 0.02)))
        pw, pw2 = tmc.pack_weights(w), tmc.pack_weights(w2)
        xin = tmc.pack_activations(x) if layout & 1 else x
        # plain GEMM (fp16 out)
        ref = torch.empty((batch, n), dtype=torch.float16, device="cuda")
        tmc.gemm_packed(x, pw, ref, n)
        y = (torch.empty(tmc.packed_activation_elements(batch, n), dtype=torch.float16,
                         device="cuda") if layout & 2 else torch.empty_like(ref))
        tmc.gemm_packed_ex(xin, pw, y, batch, k, n, layout, y_dtype=0)
        g_ref = torch.empty((batch, n), dtype=torch.float16, device="cuda")
        tmc.gate_up_silu_packed(x, pw, pw2, g_ref, n)
        g = torch.empty_like(y)
        tmc.gate_up_silu_packed_ex(xin, pw, pw2, g, batch, k, n, layout)
        torch.cuda.synchronize()
        if layout & 2:
            live = _unwritten_mask(batch, n)
            assert np.array_equal(bits(y)[live], _pack_act_reference(bits(ref))[live])
            assert np.array_equal(bits(g)[live], _pack_act_reference(bits(g_ref))[live])
        else:
            assert torch.equal(y, ref) and torch.equal(g, g_ref)
    # fp32 output with x packed
    f = torch.empty((batch, n), dtype=torch.float32, device="cuda")
    f_ref = torch.empty_like(f)
    tmc.gemm_packed(x, pw, f_ref, n)
    tmc.gemm_packed_ex(xin, pw, f, batch, k, n, layout & 1, y_dtype=1)
    torch.cuda.synchronize()
    assert torch.equal(f, f_ref)
    if layout & 2:
        with pytest.raises(tmc.TmcError):  # a packed output must be fp16
            tmc.gemm_packed_ex(xin, pw, f, batch, k, n, layout, y_dtype=1)


def test_async_raw_writes_reach_the_device_in_order(tmc, torch):
    """tmc_buf_write_raw_async: overlapping writes land in queue order, the
    caller's memory is free on return, the staging area wraps (far more than
    its 4 MiB pass through) and a copy larger than it falls back to the
    synchronous path."""
    rt = tmc.Runtime()
    n = 3 << 19  # 6 MiB of int32
    buf = rt.create_buffer(n, tmc.I32)
    rng = np.random.default_rng(77)
    expect = np.zeros(n, np.int32)
    buf.write_raw_async(expect)  # larger than the staging area
    for _ in range(300):
        count = int(rng.integers(1, 60000))
        offset = int(rng.integers(0, n - count))
        data = rng.integers(-2**31, 2**31 - 1, count, dtype=np.int32)
        expect[offset:offset + count] = data
        buf.write_raw_async(data, offset)
        data[:] = 0
    assert np.array_equal(buf.read_raw(), expect)
    with pytest.raises(tmc.TmcError):
        buf.write_raw_async(np.zeros(4, np.int32), n - 3)


def test_sparse_writes_reach_the_device_in_order(tmc, torch):
    """tmc_buf_write_sparse_async: scattered (index, value) pairs land in
    queue order with the dense staged writes around them, through enough
    calls to wrap the staging area; bad pairs are refused before anything is
    queued."""
    rt = tmc.Runtime()
    n = 1 << 20
    buf = rt.create_buffer(n, tmc.I32)
    rng = np.random.default_rng(78)
    expect = rng.integers(-2**31, 2**31 - 1, n, dtype=np.int32)
    buf.write_raw_async(expect)
    for step in range(400):
        if step % 7 == 3:  # a dense span in between
            count = int(rng.integers(1, 30000))
            offset = int(rng.integers(0, n - count))
            data = rng.integers(-2**31, 2**31 - 1, count, dtype=np.int32)
            expect[offset:offset + count] = data
            buf.write_raw_async(data, offset)
            continue
        count = int(rng.integers(1, 5000)) if step % 5 else 1
        idx = np.sort(rng.choice(n, count, replace=False)).astype(np.int32)
        if step % 11 == 0:
            idx[-1] = n - 1  # the last element
        idx = np.unique(idx)
        vals = rng.integers(-2**31, 2**31 - 1, idx.size, dtype=np.int32)
        expect[idx] = vals
        buf.write_sparse_async(idx, vals)
    assert np.array_equal(buf.read_raw(), expect)
    before = buf.read_raw()
    for idx, vals in (([3, 3], [1, 2]), ([5, 4], [1, 2]), ([n], [1]), ([-1], [1])):
        with pytest.raises(tmc.TmcError, match="indices must increase"):
            buf.write_sparse_async(idx, vals)
    with pytest.raises(tmc.TmcError, match="at most 524288 pairs"):
        buf.write_sparse_async(np.arange(524289), np.zeros(524289))
    half = rt.create_buffer(64, tmc.F16)
    with pytest.raises(tmc.TmcError, match="int32"):
        half.write_sparse_async([0], [1])
    assert np.array_equal(buf.read_raw(), before)


# ---------------------------------------------------------------- batch > 1 folded norms
@pytest.mark.parametrize("batch,k,n,layout,out_dtype", [
    (16, 4096, 4096, 1, "f16"), (5, 1160, 200, 0, "f32"), (20, 4096, 12288, 3, "f16"),
    (16, 4096, 32000, 1, "f32")])
def test_packed_gemm_with_folded_norm_matches_oracle(tmc, orc, torch, batch, k, n, layout,
                                                     out_dtype):
    """tmc_gemm_packed_norm_f16: RMSNorm(s) * gamma folded into the packed GEMM
    (weights packed as W . diag(gamma), each row scaled by its 1/rms) against
    the oracle's RMSNorm (stored fp16) followed by its linear, within the
    fp16 path tolerance (fp32 outputs too: the rounding point moves)."""
    s = orc.f16(normal(1101 + batch, (batch, k)))
    gamma = orc.f16(uniform(1102, (k,), 0.5, 1.5))
    w = orc.f16(normal(1103, (n, k), 0.02))
    pw = tmc.pack_weights(dev_f16(w), gamma=dev_f16(gamma))
    x = dev_f16(s)
    xin = tmc.pack_activations(x) if layout & 1 else x
    dt = torch.float16 if out_dtype == "f16" else torch.float32
    if layout & 2:
        y = torch.empty(tmc.packed_activation_elements(batch, n), dtype=dt, device="cuda")
    else:
        y = torch.full((batch, n), float("nan"), dtype=dt, device="cuda")
    tmc.gemm_packed_norm(xin, pw, y, batch, k, n, 1e-6, layout)
    if layout & 2:
        rm = torch.empty((batch, n), dtype=dt, device="cuda")
        tmc.pack_activations(y, rm, unpack=True, rows=batch, cols=n)
        y = rm
    torch.cuda.synchronize()
    normed = orc.f16(orc.store(orc.rmsnorm(s, gamma, F16, 1e-6), F16))
    ref = orc.linear(normed, w, F16)
    assert_f16_path(values(y), ref, what=f"folded norm GEMM b{batch} {k}->{n}")


@pytest.mark.parametrize("batch,layout", [(16, 3), (7, 1), (17, 0)])
def test_packed_gated_mlp_with_folded_norm_matches_oracle(tmc, orc, torch, batch, layout):
    k, n = 4096, 11008
    s = orc.f16(normal(1111 + batch, (batch, k)))
    gamma = orc.f16(uniform(1112, (k,), 0.5, 1.5))
    wg = orc.f16(normal(1113, (n, k), 0.02))
    wu = orc.f16(normal(1114, (n, k), 0.02))
    gd = dev_f16(gamma)
    pg, pu = tmc.pack_weights(dev_f16(wg), gamma=gd), tmc.pack_weights(dev_f16(wu), gamma=gd)
    x = dev_f16(s)
    xin = tmc.pack_activations(x) if layout & 1 else x
    if layout & 2:
        g = torch.empty(tmc.packed_activation_elements(batch, n), dtype=torch.float16,
                        device="cuda")
    else:
        g = torch.full((batch, n), float("nan"), dtype=torch.float16, device="cuda")
    tmc.gate_up_silu_packed_norm(xin, pg, pu, g, batch, k, n, 1e-6, layout)
    if layout & 2:
        rm = torch.empty((batch, n), dtype=torch.float16, device="cuda")
        tmc.pack_activations(g, rm, unpack=True, rows=batch, cols=n)
        g = rm
    torch.cuda.synchronize()
    normed = orc.f16(orc.store(orc.rmsnorm(s, gamma, F16, 1e-6), F16))
    assert_f16_path(values(g), orc.gated_mlp(normed, wg, wu, F16),
                    what=f"folded norm gated MLP b{batch}")


@pytest.mark.parametrize("batch,layout", [(16, 1), (5, 0), (17, 1)])
def test_packed_qkv_rope_append_with_folded_norm(tmc, orc, torch, batch, layout):
    """The norm-folded batched q.k.v + RoPE + append against RMSNorm (kernel)
    followed by tmc_qkv_rope_append_packed_f16: q and every written pool
    slot within the fp16 path tolerance, the same slots written (skipped
    rows, lengths outside [1, capacity] and missing pages untouched)."""
    qh, kvh, d, hidden, cap, p = 8, 4, 64, 512, 64, 16
    mp = cap // p
    pos = np.arange(cap)[:, None]
    freq = np.exp(np.arange(0, d, 2) * (-np.log(10000.0) / d))
    cos = dev(np.cos(pos * freq).astype(np.float32))
    sin = dev(np.sin(pos * freq).astype(np.float32))
    width = (qh + 2 * kvh) * d
    s = orc.f16(normal(1121 + batch, (batch, hidden)))
    gamma = dev_f16(orc.f16(uniform(1122, (hidden,), 0.5, 1.5)))
    w = dev_f16(orc.f16(normal(1123, (width, hidden), 0.05)))
    packed = tmc.pack_weights(w)
    scaled = tmc.pack_weights(w, gamma=gamma)
    x = dev_f16(s)
    xin = tmc.pack_activations(x) if layout else x
    rng = np.random.default_rng(1124)
    pages = batch * mp + 4
    tables = rng.permutation(pages)[:batch * mp].astype(np.int32).reshape(batch, mp)
    lengths = rng.integers(1, cap + 1, batch).astype(np.int32)
    lengths[0] = 0
    lengths[-1] = cap + 1
    if batch > 2:
        lengths[1] = 20
        tables[1, 1] = -1
    active = batch - 1 if batch > 2 else batch
    # NaN pools: the written slots are exactly the ones no longer NaN
    pool0 = np.full((pages, kvh, p, d), 0x7E00, np.uint16)
    args = (cos, sin, dev(lengths), dev(tables), torch.tensor([active], dtype=torch.int32,
                                                               device="cuda"))
    kp, vp = dev_f16(pool0), dev_f16(pool0.copy())
    q = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
    tmc.rmsnorm_qkv_rope_append_packed(xin, scaled, *args, q, kp, vp, batch, hidden, qh, kvh, d,
                                       cap, p, mp, 1e-6, layout)
    normed = torch.empty_like(x)
    tmc.rmsnorm(x, gamma, normed, 1e-6)
    kp2, vp2 = dev_f16(pool0), dev_f16(pool0.copy())
    q2 = torch.full_like(q, float("nan"))
    tmc.qkv_rope_append_packed(normed, packed, *args, q2, kp2, vp2, batch, hidden, qh, kvh, d, cap,
                               p, mp, 0)
    torch.cuda.synchronize()
    a, b = values(q), values(q2)
    assert np.array_equal(np.isnan(a), np.isnan(b))
    live = ~np.isnan(b)
    assert_f16_path(a[live], b[live].astype(np.float64), what="folded norm q")
    for got, want in ((kp, kp2), (vp, vp2)):
        written = ~np.isnan(values(want))
        assert written.any()
        assert np.array_equal(~np.isnan(values(got)), written)
        assert_f16_path(values(got)[written], values(want)[written].astype(np.float64),
                        what="folded norm pool slots")


@pytest.mark.parametrize("batch,k,n,layout", [(16, 4096, 4096, 2), (5, 11008, 4096, 3),
                                              (20, 4096, 4096, 0)])
def test_packed_gemm_residual_equals_gemm_then_add_bit_exact(tmc, orc, torch, batch, k, n,
                                                             layout):
    """tmc_gemm_packed_residual_f16 (emitLinearResidual over packed weights):
    the bits of tmc_gemm_packed_ex_f16 followed by tmc_add, in either
    activation layout."""
    x = dev_f16(orc.f16(normal(1131 + batch, (batch, k))))
    w = dev_f16(orc.f16(normal(1132, (n, k), 0.02)))
    res = dev_f16(orc.f16(normal(1133, (batch, n))))
    pw = tmc.pack_weights(w)
    xin = tmc.pack_activations(x) if layout & 1 else x
    resin = tmc.pack_activations(res) if layout & 2 else res
    if layout & 2:
        y = torch.empty(tmc.packed_activation_elements(batch, n), dtype=torch.float16,
                        device="cuda")
    else:
        y = torch.full((batch, n), float("nan"), dtype=torch.float16, device="cuda")
    tmc.gemm_packed_residual(xin, pw, resin, y, batch, k, n, layout)
    proj = torch.empty((batch, n), dtype=torch.float16, device="cuda")
    tmc.gemm_packed_ex(xin, pw, proj, batch, k, n, layout & 1, y_dtype=0)
    want = torch.empty_like(proj)
    tmc.add(proj, res, want)
    if layout & 2:
        rm = torch.empty((batch, n), dtype=torch.float16, device="cuda")
        tmc.pack_activations(y, rm, unpack=True, rows=batch, cols=n)
        y = rm
    torch.cuda.synchronize()
    assert np.array_equal(bits(y), bits(want))


def test_attention_timeline_build(tmc, orc, torch):
    """The build switch TMC_ATTN_TIMELINE=1 (libtmc_hip_timeline.so) stamps
    the phases of every wave of the paged split kernel (16-position pages,
    4-wave blocks) and leaves its results alone: the same bits as the plain
    library on ragged GQA-4 rows, and per live wave the stamps in order
    (entry, first step, each step's issue / arrival / end, merge, exit)."""
    batch, qh, kvh, d, p, max_pages, pages = 8, 32, 8, 128, 16, 256, 2048
    cap = p * max_pages  # 8 rows x 8 kv heads at capacity 4096: 1024-position splits
    lengths = np.array([4096, 1, 700, 2049, 1500, 3333, 64, 1025], dtype=np.int32)
    perm = np.random.default_rng(1410).permutation(pages).astype(np.int32)
    tables = np.full((batch, max_pages), -1, np.int32)
    cursor = 0
    for i, n in enumerate(lengths):
        need = (int(n) + p - 1) // p
        tables[i, :need] = perm[cursor:cursor + need]
        cursor += need
    k_d = dev_f16(orc.f16(normal(1411, (pages, kvh, p, d))))
    v_d = dev_f16(orc.f16(normal(1412, (pages, kvh, p, d))))
    q_d = dev_f16(orc.f16(normal(1413, (batch, qh * d))))
    valid_d, tables_d = dev(lengths), dev(tables)
    active = torch.tensor([batch], dtype=torch.int32, device="cuda")
    outs = []
    saved = tmc._lib
    variant = tmc.open_variant("libtmc_hip_timeline.so")
    try:
        for lib in (saved, variant):
            tmc._lib = lib
            out = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
            tmc.paged_decode_attention(q_d, k_d, v_d, valid_d, tables_d, active, out, batch, qh,
                                       kvh, d, p, max_pages, kvh * p * d, p * d,
                                       _ws(tmc, torch, batch, qh, kvh, d, cap))
            torch.cuda.synchronize()
            outs.append(bits(out))
        waves = kvh * (cap // 1024) * batch * 4  # grid (kv heads, splits, batch) x 4 waves
        events = np.zeros(waves * 48, dtype=np.uint64)
        tmc.check(variant.tmc_attention_timeline(events.ctypes.data, waves),
                  "tmc_attention_timeline")
    finally:
        tmc._lib = saved
    assert not np.isnan(outs[0].view(np.float16)).any()
    assert np.array_equal(outs[0], outs[1])
    ev = events.astype(np.int64).reshape(waves, 48)
    steps = ev[:, 8]
    live = ev[(steps > 0) & (steps < 99)]
    # the live waves: 32 positions per step, 4 waves interleaved per 1024-position split
    expect = sum(min(4, -(-(min(1024, int(n) - s) ) // 32)) for n in lengths
                 for s in range(0, int(n), 1024)) * kvh
    assert len(live) == expect
    assert (steps == 99).sum() + len(live) + ((steps == 0) & (ev[:, 0] > 0)).sum() == waves
    for w in live:
        marks = [w[3], w[9], w[4]]  # entry, unit dealt, first step
        for s in range(min(int(w[8]), 12)):
            marks += [w[10 + 3 * s], w[11 + 3 * s], w[12 + 3 * s]]
        marks += [w[5], w[6], w[7]]
        assert all(a <= b for a, b in zip(marks, marks[1:]))
        assert w[0] <= w[1]


def test_attention_merge_launch_build(tmc, orc, torch):
    """The build switch TMC_ATTN_MERGE_LAUNCH=1 (libtmc_hip_merge_launch.so)
    merges every split row in a second launch, so no block reads partials
    another block wrote in the same launch.  Its C3, C4 and workspace-reuse
    results against the oracle, as for the default build."""
    variant = tmc.open_variant("libtmc_hip_merge_launch.so")
    saved = tmc._lib
    tmc._lib = variant
    try:
        test_c3_contiguous_decode_attention(tmc, orc, torch, 4095)
        test_c4_paged_gqa_attention(tmc, orc, torch)
        test_paged_attention_workspace_reused_across_shapes(tmc, orc, torch)
    finally:
        tmc._lib = saved


@pytest.mark.parametrize("batch,qh,kvh,cap", [(16, 32, 8, 4096), (1, 32, 32, 4096),
                                              (4, 16, 8, 2048), (3, 32, 4, 4096)])
def test_merge_launch_build_equals_in_kernel_merge(tmc, orc, torch, batch, qh, kvh, cap):
    """The in-kernel merge (last-arriving split block, agent-scope stores and
    loads, no fences) against the merge launch of the TMC_ATTN_MERGE_LAUNCH=1
    build, where stream order replaces the cross-block handshake: the same
    partials merged in the same split order, so the output bits must agree.
    GQA 4 (C4's group), MHA (C3-like rows), GQA 2, and GQA 8 (merge launch in
    both builds); ragged lengths up to the capacity over random pages."""
    d, p = 128, 16
    max_pages = cap // p
    rng = np.random.default_rng(1400 + batch)
    lengths = rng.integers(1, cap + 1, size=batch).astype(np.int32)
    lengths[0] = cap
    pages = int(sum((int(n) + p - 1) // p for n in lengths)) + 3
    perm = rng.permutation(pages).astype(np.int32)
    tables = np.full((batch, max_pages), -1, np.int32)
    cursor = 0
    for i, n in enumerate(lengths):
        need = (int(n) + p - 1) // p
        tables[i, :need] = perm[cursor:cursor + need]
        cursor += need
    k_d = dev_f16(orc.f16(normal(1401, (pages, kvh, p, d))))
    v_d = dev_f16(orc.f16(normal(1402, (pages, kvh, p, d))))
    q_d = dev_f16(orc.f16(normal(1403, (batch, qh * d))))
    valid_d, tables_d = dev(lengths), dev(tables)
    active = torch.tensor([batch], dtype=torch.int32, device="cuda")
    outs = []
    saved = tmc._lib
    try:
        for lib in (saved, tmc.open_variant("libtmc_hip_merge_launch.so")):
            tmc._lib = lib
            out = torch.full((batch, qh * d), float("nan"), dtype=torch.float16, device="cuda")
            tmc.paged_decode_attention(q_d, k_d, v_d, valid_d, tables_d, active, out, batch, qh,
                                       kvh, d, p, max_pages, kvh * p * d, p * d,
                                       _ws(tmc, torch, batch, qh, kvh, d, cap))
            torch.cuda.synchronize()
            outs.append(bits(out))
    finally:
        tmc._lib = saved
    assert not np.isnan(outs[0].view(np.float16)).any()
    assert np.array_equal(outs[0], outs[1])


# ---------------------------------------------------------------- token-only LM head
def _lm_head_inputs(orc, batch, k, vocab, seed):
    """Residual rows, gamma and an LM head W with planted duplicates: rows 5
    and vocab - 1 equal row 17 (exact ties of the same logit), and row 9
    holds an fp16 NaN (its logit is NaN and is never selected)."""
    s = orc.f16(normal(seed, (batch, k)))
    gamma = orc.f16(uniform(seed + 1, (k,), 0.5, 1.5))
    w = orc.f16(normal(seed + 2, (vocab, k), 0.02))
    w[5] = w[17]
    w[vocab - 1] = w[17]
    w[9, 3] = 0x7E00  # NaN
    return s, gamma, w


@pytest.mark.parametrize("vocab", [32000, 4099, 5])
def test_lm_head_token_only_batch1(tmc, orc, torch, vocab):
    """tmc_rmsnorm_lm_head_partial_argmax_f16 + tmc_lm_head_final_argmax
    equal the logits path (tmc_add_rmsnorm_gemv_f16, fp32 logits, then
    tmc_argmax_f32) token for token, ties to the lowest index and NaN never
    chosen; with row 17's logit raised to the maximum, rows 5, 17 and
    vocab - 1 tie and the token is 5.  Against the oracle: the token is the
    oracle's argmax over its own logits."""
    k = 4096
    s, gamma, w = _lm_head_inputs(orc, 1, k, max(vocab, 18), 1300)
    w = w[:vocab]
    s_values = np.asarray(s[0], np.uint16).view(np.float16).astype(np.float32)
    ws = torch.zeros(tmc.lm_head_argmax_workspace_bytes(1, vocab) // 4, dtype=torch.float32,
                     device="cuda")
    for boost in (False, True):
        wb = w.copy()
        if boost and vocab >= 18:
            wb[[5, 17, vocab - 1]] = orc.f16(0.05 * np.sign(s_values))
        wd = dev_f16(wb)
        logits = torch.empty((1, vocab), dtype=torch.float32, device="cuda")
        tmc.add_rmsnorm_gemv(dev_f16(s), None, dev_f16(gamma), wd, None, logits, 1e-6)
        ref_tok = torch.empty(1, dtype=torch.int32, device="cuda")
        tmc.argmax(logits, ref_tok)
        tok = torch.full((1,), -7, dtype=torch.int32, device="cuda")
        tmc.rmsnorm_lm_head_argmax(dev_f16(s), dev_f16(gamma), wd, ws, tok, 1e-6)
        torch.cuda.synchronize()
        got = int(tok.cpu()[0])
        assert got == int(ref_tok.cpu()[0]), (vocab, boost)
        assert got != 9
        if boost and vocab >= 18:
            assert got == 5
        # the oracle: its argmax, unless its top two logits are within the
        # fp16-path tolerance (2e-2) and the chosen token is one of them
        normed = orc.f16(orc.store(orc.rmsnorm(s, gamma, F16, 1e-6), F16))
        ref_logits = orc.linear(normed, wb, F16)[0]
        ref = int(orc.argmax(ref_logits[None, :])[0])
        finite = np.where(np.isnan(ref_logits), -np.inf, ref_logits)
        if got != ref:
            gap = finite[ref] - finite[got]
            assert gap <= 2e-2, (vocab, boost, got, ref, gap)


@pytest.mark.parametrize("batch,layout", [(16, 1), (16, 0), (5, 1), (20, 1)])
def test_lm_head_token_only_packed(tmc, orc, torch, batch, layout):
    """tmc_lm_head_partial_argmax_packed_norm_f16 + the final argmax equal
    tmc_gemm_packed_norm_f16 (fp32 logits) + tmc_argmax_f32 row by row at
    V = 32000, with planted ties (rows 5, 17, 31999 equal) and a NaN row;
    batches of one, a part of, and more than one 16-row pass."""
    k, vocab = 4096, 32000
    s, gamma, w = _lm_head_inputs(orc, batch, k, vocab, 1310 + batch)
    pw = tmc.pack_weights(dev_f16(w), gamma=dev_f16(gamma))
    x = dev_f16(s)
    xin = tmc.pack_activations(x) if layout else x
    logits = torch.empty((batch, vocab), dtype=torch.float32, device="cuda")
    tmc.gemm_packed_norm(xin, pw, logits, batch, k, vocab, 1e-6, layout)
    ref_tok = torch.empty(batch, dtype=torch.int32, device="cuda")
    tmc.argmax(logits, ref_tok)
    ws = torch.zeros(tmc.lm_head_argmax_workspace_bytes(batch, vocab) // 4, dtype=torch.float32,
                     device="cuda")
    tok = torch.full((batch,), -7, dtype=torch.int32, device="cuda")
    tmc.lm_head_argmax_packed_norm(xin, pw, ws, tok, batch, k, vocab, 1e-6, layout)
    torch.cuda.synchronize()
    got = tok.cpu().numpy()
    assert list(got) == list(ref_tok.cpu().numpy())
    assert 9 not in got
    # ties: where row 17's logit is a row's maximum, the token is 5
    lg = logits.cpu().numpy()
    for r in range(batch):
        if lg[r, 17] >= np.nanmax(lg[r]):
            assert got[r] == 5
