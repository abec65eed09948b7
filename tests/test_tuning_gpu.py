"""GPU: the tuners and admission paths end to end on gfx950 — every admitted
or fallback selection must reproduce the oracle (DecodeGEMVTuner.cpp:162-304,
RMSNormTuner.cpp:159-309, DecoderLLMExecutor.cpp:92-163,
GeneratedKernelAdmission.cpp:204-318)."""
import json

import numpy as np
import pytest

from tests.helpers import F16, F32, assert_f16_path, assert_f32_rel, dev_f16, normal, uniform, values

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    if not t.cuda.is_available():
        pytest.skip("no GPU")
    return t


@pytest.fixture(scope="module")
def rt(host, torch):
    runtime = host.HipRuntime()
    assert runtime.is_available(), runtime.initialization_error()
    return runtime


@pytest.mark.parametrize("batch,k,n", [(1, 4096, 4096), (8, 1024, 2048)])
def test_tune_decode_gemv_selects_a_correct_faster_config(tmc, orc, host, rt, torch, batch, k, n):
    x = orc.f16(normal(600 + batch, (batch, k)))
    w = orc.f16(normal(601, (n, k), 0.02))
    r = host.tune_decode_gemv(rt, batch, k, n, orc.f16_values(x).ravel(),
                              orc.f16_values(w).ravel())
    assert r["success"], r["error"] + r["log"]
    # the one-thread-per-output baseline is far slower than the gfx950 kernels
    assert not r["use_baseline"], r["log"]
    assert r["speedup"] >= 1.05
    assert "Hardware Filter" in r["log"] or r["log"].count("admitted") >= 1
    # the selected configuration reproduces the oracle
    cfg = tmc.GemvConfig(*r["config"])
    y = torch.empty((batch, n), dtype=torch.float32, device="cuda")
    tmc.gemv_config(dev_f16(x), dev_f16(w), y, cfg)
    torch.cuda.synchronize()
    assert_f32_rel(values(y), orc.linear(x, w, F16), what=f"tuned {r['config']}")


@pytest.mark.parametrize("rows,width,f16", [(1, 4096, False), (3, 4097, False), (16, 4096, True)])
def test_tune_rms_norm(orc, host, rt, rows, width, f16):
    x = normal(610, (rows, width))
    if rows > 1:
        x[1] *= 1e-4
    gamma = uniform(611, (width,), 0.5, 1.5)
    if f16:
        x, gamma = orc.f16(x), orc.f16(gamma)  # bits; the host takes their values
    r = host.tune_rms_norm(rt, rows, width, 1e-6, f16,
                           (orc.f16_values(x) if f16 else x).ravel(),
                           orc.f16_values(gamma) if f16 else gamma)
    assert r["success"], r["error"] + r["log"]
    assert r["selected_threads"] in (64, 128, 256, 512, 1024)
    assert len(r["candidates"]) == 5
    for c in r["candidates"]:
        # every candidate passed correctness; admission is timing only
        assert c["outcome"] in ("Admitted", "Compare Baseline FAIL"), c
    out = np.asarray(r["output"]).reshape(rows, width)
    ref = orc.rmsnorm(x, gamma, F16 if f16 else F32, 1e-6)
    if f16:
        assert_f16_path(out, ref, what="tuned rmsnorm fp16")
    else:
        assert_f32_rel(out, ref, what="tuned rmsnorm fp32")


def test_admit_add_rmsnorm_fusion(orc, host, rt):
    rows, width = 4, 4096
    d = host.admit_add_rmsnorm_fusion(rt, rows, width, True)
    assert "Fusion AddRMSNorm" in d["log"]
    assert "error:" not in d["log"], d["log"]        # validation and timing ran
    # the second call reuses the cached decision
    assert d["cached_admitted"] == d["admitted"]
    assert "cached" in d["log"]
    assert d["steps"] == (1 if d["admitted"] else 2)
    # the buffers hold the last candidate validation run on the test inputs
    i = np.arange(rows * width)
    test = (((i % 31) - 15) / 31.0).astype(np.float32).reshape(rows, width)
    h = orc.f16(test)
    gamma = orc.f16((0.5 + (np.arange(width) % 11) / 10.0).astype(np.float32))
    s_ref, n_ref = orc.add_rmsnorm(h, h, gamma, F16, 1e-6)
    assert_f16_path(np.asarray(d["sum"]).reshape(rows, width), s_ref, what="fused sum")
    assert_f16_path(np.asarray(d["norm"]).reshape(rows, width), n_ref, what="fused norm")


def _response(tmp_path, **fields):
    path = tmp_path / "response.json"
    path.write_text(json.dumps(fields))
    return str(path)


def test_admit_generated_kernel_outcomes(host, rt, tmp_path):
    fb = tmp_path / "feedback.json"
    art = tmp_path / "admitted.json"
    # a legal candidate: correctness passes; admission depends on timing
    ok, log = host.admit_generated_kernel(
        rt, "RMSNorm",
        _response(tmp_path, function_name="rmsnorm",
                  source="rmsnorm?rows=1&width=4096&eps=1e-06&dtype=f16&threads=512",
                  workgroup_size=512),
        str(fb), str(art))
    feedback = json.loads(fb.read_text())
    assert ok, log
    assert feedback["version"] == 1
    assert feedback["status"] in ("admitted", "retry"), feedback
    assert feedback["stage"] in ("admission", "performance"), feedback
    assert feedback["metrics"] is not None and feedback["metrics"]["speedup"] > 0
    assert art.exists() == (feedback["status"] == "admitted")
    # wrong function name -> retry at the contract stage
    ok, _ = host.admit_generated_kernel(
        rt, "AddRMSNorm",
        _response(tmp_path, function_name="rmsnorm", source="rmsnorm?threads=256",
                  workgroup_size=256), str(fb))
    assert ok and json.loads(fb.read_text())["stage"] == "contract"
    # illegal workgroup -> retry at the hardware filter
    ok, _ = host.admit_generated_kernel(
        rt, "SiLUMul",
        _response(tmp_path, function_name="silu_mul", source="silu_mul?count=1",
                  workgroup_size=96), str(fb))
    assert ok and json.loads(fb.read_text())["stage"] == "hardware_filter"
    # a key the runtime rejects -> retry at compile
    ok, _ = host.admit_generated_kernel(
        rt, "RMSNorm",
        _response(tmp_path, function_name="rmsnorm", source="rmsnorm?variant=fastest",
                  workgroup_size=256), str(fb))
    assert ok and json.loads(fb.read_text())["stage"] == "compile"
    # an unknown pattern is fatal
    ok, _ = host.admit_generated_kernel(rt, "Softmax", _response(tmp_path), str(fb))
    assert not ok and json.loads(fb.read_text())["status"] == "fatal"


def test_registry_artifact_drives_the_decoder_norms(host, orc, rt, tmp_path):
    """An admitted Add+RMSNorm artifact (KernelRegistry, written as
    admitGeneratedKernel writes it) is loaded by compileDecoderLLM through
    kernel_library and replaces the template launch parameters of the
    one-row bucket's residual norms; the decode step still matches the
    oracle, and the usage audit counts the generated dispatches."""
    from tests.test_decoder_gpu import P, OracleRequest, _weights, _workload, assert_f16_path
    cfg = dict(layers=1, hidden=4096, heads=32, head_dim=128, kv_heads=8, intermediate=512,
               vocabulary=1000, capacity=64, epsilon=1e-6)
    m = _weights(orc, cfg, 81)
    w = _workload(host, orc, cfg, m)
    lib = tmp_path / "lib"
    err = host.write_admitted_kernel(rt, "AddRMSNorm", "add_rmsnorm",
                                     "add_rmsnorm?rows=1&width=4096&eps=1e-06&dtype=f16&threads=256",
                                     256, str(lib / "decoder_residual_rmsnorm" / "admitted.json"))
    assert err == ""
    opts = host.DecoderLLMCompileOptions()
    opts.kv_page_size = P
    opts.kernel_library = str(lib)
    dec, log = host.compile_decoder_llm(rt, w, opts)
    assert "decoder_residual_rmsnorm: admitted" in log, log
    prompt = [float(t) for t in np.random.default_rng(82).integers(0, cfg["vocabulary"], 5)]
    res = dec.prefill(prompt, True)
    assert res["passed"], res["error"]
    report = dec.kernel_usage_report()
    assert "generated add_rmsnorm?" in report and "threads=256" in report, report
    assert "entry decoder_residual_rmsnorm: ran" in report, report
    # 5 one-row steps x 2 residual norms per layer (1 layer)
    assert "5 calls, 10 dispatches" in report, report
    ref = OracleRequest(orc, cfg, m, cfg["capacity"] // P)
    tables = [dec.kv_block_table(l) for l in range(cfg["layers"])]
    V = cfg["vocabulary"]
    for i, tok in enumerate(prompt):
        logits, _ = ref.step(int(tok), i + 1, tables)
        assert_f16_path(res["logits"][i * V:(i + 1) * V], logits, f"position {i}")
