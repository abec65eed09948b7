"""GPU: imported `.tmc` workloads run end to end on the gfx950 path, as the
reference's decoder_llm_main.cpp / kv_cache_main.cpp run them, and match the
references the manifest carries (written by tests/tmc_manifest.py from the
oracle's decoder step and a float64 restatement of the KV-cache attention
module).

Tolerances: fp16-path values within 2e-2 absolute and 3e-3 relative RMS;
greedy tokens equal unless the reference's top two logits are within that
tolerance."""
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
