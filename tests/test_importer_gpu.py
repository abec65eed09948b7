"""GPU: imported `.tmc` workloads run end to end on the gfx950 path, as the
reference's decoder_llm_main.cpp / kv_cache_main.cpp run them, and match the
references the manifest carries (written by tests/tmc_manifest.py from the
oracle's decoder step and a float64 restatement of the KV-cache attention
module).

Tolerances: fp16-path values within 2e-2 absolute and 3e-3 relative RMS;
greedy tokens equal unless the reference's top two logits are within that
tolerance."""
import os

import numpy as np
import pytest

from tests import tmc_manifest as tm
from tests.helpers import assert_f16_path, dev, dev_f16, values

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    if not t.cuda.is_available():
        pytest.skip("no GPU")
    return t


@pytest.fixture(scope="module")
def rt(host, torch):
    r = host.HipRuntime()
    assert r.is_available(), r.initialization_error()
    return r


def _token(gpu, ref_token, ref_logits, what):
    if gpu != ref_token:
        top = np.sort(np.asarray(ref_logits))[-2:]
        assert top[1] - top[0] <= 2e-2, f"{what}: token {gpu} != {ref_token}"


CASES = {
    # the reference exporter's default shape (head_dim 16): stepped prefill
    "default": (tm.decoder_config(), 0),
    # head_dim 128: chunked prefill in chunks of 16 as well
    "d128": (tm.decoder_config(hidden=256, heads=2, inter=256, vocab=256, capacity=64, prefill=24,
                               decode=6), 16),
}


@pytest.mark.parametrize("name", list(CASES))
def test_imported_decoder_matches_manifest(host, orc, rt, tmp_path, name):
    config, chunk = CASES[name]
    tensors = tm.decoder_tensors(orc, config, seed=11)
    path = tm.write_decoder_manifest(tmp_path / "decoder_llm.tmc", config, tensors)
    workload, err = host.import_decoder_llm_workload(str(path))
    assert err == "", err
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = 16
    opts.prefill_chunk_size = chunk
    dec, _ = host.compile_decoder_llm(rt, workload, opts)
    V, L, P = config["vocabulary_size"], config["layers"], config["prefill_length"]
    D = config["hidden_size"] // config["heads"]
    ref = workload.prefill
    runs = ["prefill"] + (["prefill_chunked"] if chunk else [])
    for run in runs:
        assert dec.reset() == ""
        out = getattr(dec, run)([float(t) for t in ref.token_ids], True)
        assert out["passed"], out["error"]
        assert_f16_path(out["logits"], ref.logits, what=f"{name} {run} logits")
        _token(int(out["next_token_ids"][-1]), int(ref.next_token_ids[0]),
               ref.logits.reshape(P, V)[-1], f"{name} {run} token")
        for l in range(L):
            assert_f16_path(dec.read_key_prefix(l), ref.key_caches[l], what=f"{name} {run} K{l}")
            assert_f16_path(dec.read_value_prefix(l), ref.value_caches[l],
                            what=f"{name} {run} V{l}")
    for s, step in enumerate(workload.decode_steps):
        out = dec.decode([float(step.token_ids[0])], True)
        assert out["passed"], out["error"]
        assert_f16_path(out["logits"], step.logits, what=f"{name} decode {s} logits")
        _token(int(out["next_token_ids"][0]), int(step.next_token_ids[0]), step.logits,
               f"{name} decode {s} token")
        for l in range(L):
            assert dec.read_key_prefix(l).size == config["heads"] * (P + s + 1) * D
            assert_f16_path(dec.read_value_prefix(l), step.value_caches[l],
                            what=f"{name} decode {s} V{l}")


def test_imported_kv_workload_on_gfx950_kernels(host, tmc, orc, rt, tmp_path, torch):
    """The KV-cache attention module (projections, cache append, attention
    over every cached position, o projection) composed from the backend's
    kernels: gemm_rows, kv_append, paged decode attention over the cache as
    one page (one row per query token, all sharing it) and gemm_rows."""
    config, tensors, steps = tm.kv_workload(7)
    path = tm.write_kv_manifest(tmp_path / "kv_cache.tmc", config, tensors, steps)
    w, err = host.import_kv_cache_workload(str(path))
    assert err == "", err
    heads, d, cap = w.plan.heads, w.plan.head_dimension, w.plan.capacity
    dim = heads * d
    f16 = lambda a: dev_f16(orc.f16(np.asarray(a, np.float32).reshape(-1, dim)))  # noqa: E731
    wq, wk, wv, wo = (f16(x) for x in (w.query_weight, w.key_weight, w.value_weight, w.output_weight))
    k_cache = torch.zeros((heads, cap, d), dtype=torch.float16, device="cuda")
    v_cache = torch.zeros_like(k_cache)

    def run(step, start):
        xq, xk, xv = (f16(x) for x in (step.query, step.key, step.value))
        rows = xq.shape[0]
        proj = []
        for x, wt in ((xq, wq), (xk, wk), (xv, wv)):
            y = torch.empty((rows, dim), dtype=torch.float16, device="cuda")
            tmc.gemm_rows(x, wt, y)
            proj.append(y)
        length = torch.tensor([start + rows], dtype=torch.int32, device="cuda")
        tmc.kv_append(proj[1], length, k_cache, 1, rows, heads, d, cap, False)
        tmc.kv_append(proj[2], length, v_cache, 1, rows, heads, d, cap, False)
        lengths = dev(np.full(rows, start + rows, np.int32))
        tables = dev(np.zeros((rows, 1), np.int32))
        ctx = torch.full((rows, dim), float("nan"), dtype=torch.float16, device="cuda")
        ws_bytes = tmc.attention_workspace_bytes(rows, heads, heads, d, cap)
        ws = torch.zeros(max(ws_bytes // 4, 1), dtype=torch.float32, device="cuda")
        tmc.paged_decode_attention(proj[0], k_cache, v_cache, lengths,
                                   tables, torch.tensor([rows], dtype=torch.int32, device="cuda"),
                                   ctx, rows, heads, heads, d, cap, 1, heads * cap * d, cap * d,
                                   ws if ws_bytes else None)
        out = torch.empty((rows, dim), dtype=torch.float16, device="cuda")
        tmc.gemm_rows(ctx, wo, out)
        torch.cuda.synchronize()
        return values(out)

    got = run(w.prefill, 0)
    assert_f16_path(got, w.prefill.output, what="KV prefill output")
    P = w.plan.prefill_length
    assert_f16_path(values(k_cache)[:, :P], w.prefill.key_cache, what="KV prefill key cache")
    for s, step in enumerate(w.decode_steps):
        got = run(step, P + s)
        assert_f16_path(got, step.output, what=f"KV decode {s} output")
        n = P + s + 1
        assert_f16_path(values(v_cache)[:, :n], step.value_cache, what=f"KV decode {s} value cache")


GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.mark.parametrize("fixture", ["decoder_llm_fp16_seed11.tmc", "decoder_llm_fp32_seed11.tmc"])
def test_reference_exported_decoder(host, orc, rt, fixture):
    """A manifest written by the reference's own exporter
    (tools/export_decoder_llm.py --seed 11 at its default shape, fp16 and
    fp32; tests/golden/make_tmc_golden.py) imported and run through
    compileDecoderLLM as decoder_llm_main.cpp runs it: prefill, then each
    decode step's token.  Logits and K/V prefixes against the PyTorch
    references in the manifest at the reference app's fp16 tolerance
    (Validator::compare, 2e-2 absolute + 2e-2 relative,
    decoder_llm_main.cpp:15-23; the fp32 manifest too, since this decoder
    stores fp16), tokens equal unless the reference's top two logits are
    within 2e-2; and every logit against the oracle's decoder step on the
    same fp16 weights at the fp16-path tolerance."""
    workload, err = host.import_decoder_llm_workload(os.path.join(GOLDEN, fixture))
    assert err == "", err
    plan = workload.plan
    assert (plan.layer_count, plan.attention.heads, plan.attention.head_dimension,
            plan.vocabulary_size, plan.attention.prefill_length) == (2, 4, 16, 128, 8)
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = 16
    dec, _ = host.compile_decoder_llm(rt, workload, opts)
    V, L, P = plan.vocabulary_size, plan.layer_count, plan.attention.prefill_length
    ref = workload.prefill
    decode_tokens = [int(s.token_ids[0]) for s in workload.decode_steps]
    oracle = tm.oracle_decoder_run(orc, workload, [int(t) for t in ref.token_ids], decode_tokens)

    def check(what, logits, reference, oracle_logits):
        ok, worst, mismatches = orc.compare(logits, reference, 2e-2, 2e-2)
        assert ok, f"{what}: {mismatches} logits outside 2e-2 + 2e-2 |ref| (worst {worst:.3e})"
        assert_f16_path(logits, oracle_logits, what=f"{what} against the oracle")

    out = dec.prefill([float(t) for t in ref.token_ids], True)
    assert out["passed"], out["error"]
    check(f"{fixture} prefill", out["logits"], ref.logits, oracle[0][0])
    _token(int(out["next_token_ids"][-1]), int(ref.next_token_ids[0]),
           ref.logits.reshape(P, V)[-1], f"{fixture} prefill token")
    for l in range(L):
        for got, want in ((dec.read_key_prefix(l), ref.key_caches[l]),
                          (dec.read_value_prefix(l), ref.value_caches[l])):
            ok, worst, _ = orc.compare(got, want, 2e-2, 2e-2)
            assert ok, f"{fixture} prefill cache layer {l}: worst {worst:.3e}"
        assert_f16_path(dec.read_key_prefix(l), oracle[0][2][l], what=f"prefill K{l} vs oracle")
    for s, step in enumerate(workload.decode_steps):
        out = dec.decode([float(step.token_ids[0])], True)
        assert out["passed"], out["error"]
        check(f"{fixture} decode {s}", out["logits"], step.logits, oracle[s + 1][0])
        _token(int(out["next_token_ids"][0]), int(step.next_token_ids[0]), step.logits,
               f"{fixture} decode {s} token")
        for l in range(L):
            ok, worst, _ = orc.compare(dec.read_value_prefix(l), step.value_caches[l], 2e-2, 2e-2)
            assert ok, f"{fixture} decode {s} V{l}: worst {worst:.3e}"
            assert_f16_path(dec.read_value_prefix(l), oracle[s + 1][3][l],
                            what=f"decode {s} V{l} vs oracle")
    assert dec.current_length() == P + len(workload.decode_steps)


def test_reference_exported_kv_cache(host, orc, rt):
    """The reference exporter's KV-cache manifest (tools/export_kv_cache.py,
    MultiHeadAttentionKVCache: 4 heads x 16, prefill 7, 8 decode steps)
    through compileKVCacheAttention as kv_cache_main.cpp runs it.  The
    reference module is fp32 and its app checks 2e-4 + 2e-3 |ref|
    (kv_cache_main.cpp:15-16); this module stores fp16 (inputs rounded on
    upload), so outputs and caches are held to the fp16-path tolerance and
    to the reference app's fp16 bound (2e-2 + 2e-2 |ref|)."""
    w, err = host.import_kv_cache_workload(os.path.join(GOLDEN, "kv_cache.tmc"))
    assert err == "", err
    plan = w.plan
    assert (plan.batch, plan.heads, plan.head_dimension, plan.capacity, plan.prefill_length) == \
        (1, 4, 16, 15, 7)
    exe, _ = host.compile_kv_cache_attention(rt, plan, w.query_weight, w.key_weight,
                                             w.value_weight, w.output_weight)

    def check(what, got, want):
        ok, worst, _ = orc.compare(got, want, 2e-2, 2e-2)
        assert ok, f"{what}: worst {worst:.3e}"
        assert_f16_path(got, want, what=what)

    out = exe.prefill(w.prefill.query, w.prefill.key, w.prefill.value)
    assert out["passed"], out["error"]
    check("prefill output", out["output"], w.prefill.output)
    check("prefill key cache", exe.read_key_prefix(), w.prefill.key_cache)
    check("prefill value cache", exe.read_value_prefix(), w.prefill.value_cache)
    for s, step in enumerate(w.decode_steps):
        out = exe.decode(step.query, step.key, step.value)
        assert out["passed"], out["error"]
        check(f"decode {s} output", out["output"], step.output)
        check(f"decode {s} key cache", exe.read_key_prefix(), step.key_cache)
        check(f"decode {s} value cache", exe.read_value_prefix(), step.value_cache)
    assert exe.current_length() == plan.capacity
