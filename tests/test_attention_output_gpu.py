"""GPU parity of the batch-1 paged attention + output projection fusion
(tmc_paged_attention_output_f16; reference: emitPagedAttentionOutputProjection,
DecoderLLMMetalEmitter.cpp:623-698, with the residual add of
emitLinearResidual, :604-621) against the CPU oracle: the oracle's paged
attention, rounded to fp16 as the attention kernel stores it, through the
oracle's linear, plus the residual.  Also checked: the output is the same
bits on every call (the kv heads' partial sums are added in head order
whichever block arrives last, and each call leaves the arrival counters at
zero), and rows the attention kernel leaves untouched stay untouched."""
import numpy as np
import pytest

from tests.helpers import F16, assert_f16_path, bits, dev, dev_f16, normal, values

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


def _case(orc, seed, qh, kvh, p, max_pages, pool, out, lengths):
    d = 128
    rng = np.random.default_rng(seed)
    k_pool = orc.f16(normal(seed + 1, (pool, kvh, p, d)))
    v_pool = orc.f16(normal(seed + 2, (pool, kvh, p, d)))
    q = orc.f16(normal(seed + 3, (1, qh * d)) * 2)
    w = orc.f16(normal(seed + 4, (out, qh * d), 0.02))
    res = orc.f16(normal(seed + 5, (1, out)))
    table = np.full((1, max_pages), -1, np.int32)
    table[0] = rng.permutation(pool)[:max_pages]
    return k_pool, v_pool, q, w, res, table


def _reference(orc, q, k_pool, v_pool, w, res, table, qh, kvh, p, max_pages, length):
    d = 128
    ctx, written = orc.paged_attention(q, k_pool, v_pool, F16, qh, kvh, d, p, kvh * p * d, p * d,
                                       table, max_pages, np.array([length], np.int32), 1)
    assert written.all()
    proj = orc.store(orc.linear(orc.f16(ctx), w, F16), F16)
    return proj if res is None else orc.f16_values(res).astype(np.float64) + proj


def _run(tmc, torch, q_d, k_d, v_d, len_d, table_d, active, w_d, res_d, y, qh, kvh, p, max_pages,
         ws):
    tmc.paged_attention_output(q_d, k_d, v_d, len_d, table_d, active, w_d, res_d, y, qh, kvh, 128,
                               p, max_pages, kvh * p * 128, p * 128, ws)


def _counters_clear(ws):
    """The workspace's arrival counters (its first 256 bytes here) are zero."""
    return not ws[:64].cpu().numpy().any()


def _workspace(tmc, torch, qh, kvh, out):
    n = tmc.attention_output_workspace_bytes(qh, kvh, out)
    assert n > 0
    return torch.zeros(n // 4, dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("qh,kvh,p,max_pages,pool,out,lengths", [
    # Llama-7B widths (32 heads x 128, hidden 4096): 8 slices of 512 rows per
    # kv head, slices of one head on one XCD
    (32, 32, 16, 64, 96, 4096, (1, 77, 260, 1024)),
    # GQA group 2: 256-row slices
    (8, 4, 32, 8, 12, 512, (200, 256)),
    # 4 kv heads (no XCD grouping), 128-row slices (3 per head), pages of
    # 48 positions (not a power of two)
    (4, 4, 48, 21, 24, 384, (1000, 48, 49)),
])
def test_attention_output_matches_oracle_and_repeats(tmc, orc, torch, qh, kvh, p, max_pages, pool,
                                                     out, lengths):
    k_pool, v_pool, q, w, res, table = _case(orc, 900 + qh + p, qh, kvh, p, max_pages, pool, out,
                                             lengths)
    k_d, v_d, q_d, w_d, res_d = dev_f16(k_pool), dev_f16(v_pool), dev_f16(q), dev_f16(w), dev_f16(res)
    table_d = dev(table)
    active = torch.tensor([1], dtype=torch.int32, device="cuda")
    ws = _workspace(tmc, torch, qh, kvh, out)
    y = torch.empty((1, out), dtype=torch.float16, device="cuda")
    for length in lengths:
        len_d = torch.tensor([length], dtype=torch.int32, device="cuda")
        first = None
        for call in range(3):
            y.fill_(float("nan"))
            _run(tmc, torch, q_d, k_d, v_d, len_d, table_d, active, w_d, res_d, y, qh, kvh, p,
                 max_pages, ws)
            torch.cuda.synchronize()
            got = bits(y)
            if first is None:
                first = got
                ref = _reference(orc, q, k_pool, v_pool, w, res, table, qh, kvh, p, max_pages,
                                 length)
                assert_f16_path(values(y), ref, what=f"qh{qh} kvh{kvh} p{p} L{length}")
            else:
                assert np.array_equal(got, first), f"call {call} differs (L{length})"
        # every call leaves the counters at zero
        assert _counters_clear(ws), ws[:64].cpu().numpy()


def test_attention_output_without_residual_and_against_two_kernels(tmc, orc, torch):
    """residual NULL stores fp16(W . context); with the residual the result
    is within the fp16 path tolerance of the two-kernel path (attention
    kernel, then the residual GEMV)."""
    qh = kvh = 32
    p, max_pages, pool, out, length = 16, 64, 80, 4096, 333
    k_pool, v_pool, q, w, res, table = _case(orc, 950, qh, kvh, p, max_pages, pool, out, ())
    k_d, v_d, q_d, w_d, res_d = dev_f16(k_pool), dev_f16(v_pool), dev_f16(q), dev_f16(w), dev_f16(res)
    table_d = dev(table)
    len_d = torch.tensor([length], dtype=torch.int32, device="cuda")
    ws = _workspace(tmc, torch, qh, kvh, out)
    y = torch.full((1, out), float("nan"), dtype=torch.float16, device="cuda")
    _run(tmc, torch, q_d, k_d, v_d, len_d, table_d, None, w_d, None, y, qh, kvh, p, max_pages, ws)
    torch.cuda.synchronize()
    ref = _reference(orc, q, k_pool, v_pool, w, None, table, qh, kvh, p, max_pages, length)
    assert_f16_path(values(y), ref, what="no residual")

    y_res = torch.full((1, out), float("nan"), dtype=torch.float16, device="cuda")
    _run(tmc, torch, q_d, k_d, v_d, len_d, table_d, None, w_d, res_d, y_res, qh, kvh, p, max_pages,
         ws)
    ctx = torch.full((1, qh * 128), float("nan"), dtype=torch.float16, device="cuda")
    tmc.paged_decode_attention(q_d, k_d, v_d, len_d, table_d, None, ctx, 1, qh, kvh, 128, p,
                               max_pages, kvh * p * 128, p * 128)
    two = torch.full((1, out), float("nan"), dtype=torch.float16, device="cuda")
    tmc.gemv_residual(ctx, w_d, res_d, two)
    torch.cuda.synchronize()
    assert_f16_path(values(y_res), values(two).astype(np.float64), what="fused vs two kernels")


def test_attention_output_leaves_skipped_rows_untouched(tmc, orc, torch):
    """An inactive request, an invalid length and a missing page (negative or
    past the pool) leave y untouched, as the attention kernel leaves its
    output; the next valid call is still exact (the counters were reset)."""
    qh = kvh = 8
    p, max_pages, pool, out = 16, 16, 20, 512
    k_pool, v_pool, q, w, res, table = _case(orc, 960, qh, kvh, p, max_pages, pool, out, ())
    k_d, v_d, q_d, w_d, res_d = dev_f16(k_pool), dev_f16(v_pool), dev_f16(q), dev_f16(w), dev_f16(res)
    ws = _workspace(tmc, torch, qh, kvh, out)
    y = torch.empty((1, out), dtype=torch.float16, device="cuda")
    holes = table.copy()
    holes[0, 2] = -1
    past = table.copy()
    past[0, 1] = pool + 5
    cases = [("inactive", table, 40, 0), ("length 0", table, 0, 1),
             ("length past capacity", table, p * max_pages + 1, 1), ("hole", holes, 40, 1),
             ("page past pool", past, 40, 1)]
    for what, tab, length, act in cases:
        y.fill_(float("nan"))
        _run(tmc, torch, q_d, k_d, v_d, torch.tensor([length], dtype=torch.int32, device="cuda"),
             dev(tab), torch.tensor([act], dtype=torch.int32, device="cuda"), w_d, res_d, y, qh,
             kvh, p, max_pages, ws)
        torch.cuda.synchronize()
        assert torch.isnan(y).all(), what
    assert _counters_clear(ws), ws[:64].cpu().numpy()
    y.fill_(float("nan"))
    _run(tmc, torch, q_d, k_d, v_d, torch.tensor([40], dtype=torch.int32, device="cuda"),
         dev(table), torch.tensor([1], dtype=torch.int32, device="cuda"), w_d, res_d, y, qh, kvh, p,
         max_pages, ws)
    torch.cuda.synchronize()
    ref = _reference(orc, q, k_pool, v_pool, w, res, table, qh, kvh, p, max_pages, 40)
    assert_f16_path(values(y), ref, what="valid call after skipped ones")
