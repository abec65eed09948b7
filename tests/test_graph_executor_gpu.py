"""GPU: compileGraph on the gfx950 backend (GraphExecutor.cpp:346-430):
RMSNorm tuning, fusion-region admission and execution of TensorIR graphs,
outputs against the pinned oracle."""
import numpy as np
import pytest

from tests.helpers import F16, F32, assert_f16_path, assert_f32_rel, normal, uniform
from tests.test_graph_executor import _mlp_graph

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt(host):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    runtime = host.HipRuntime()
    assert runtime.is_available(), runtime.initialization_error()
    return runtime


@pytest.mark.parametrize("rows", [1, 8])
def test_c2_graph_compiles_tunes_and_matches_oracle(host, orc, rt, rows):
    """C2's MLP block at full size (hidden 4096, intermediate 11008) as a
    TensorIR graph: two fusion regions are tuned and decided, the RMSNorm is
    tuned, and the output matches the oracle."""
    hidden, inter = 4096, 11008
    g, ids = _mlp_graph(host, rows, hidden, inter, host.DType.Float16)
    h, r = normal(920 + rows, (rows, hidden)), normal(921 + rows, (rows, hidden))
    gamma = uniform(922, (hidden,), 0.5, 1.5)
    wg, wu = normal(923, (inter, hidden), 0.02), normal(924, (inter, hidden), 0.02)
    wd = normal(925, (hidden, inter), 0.02)
    c = host.compile_graph(rt, g, {ids["h"]: h.ravel(), ids["r"]: r.ravel(), ids["gamma"]: gamma,
                                   ids["wg"]: wg.ravel(), ids["wu"]: wu.ravel(),
                                   ids["wd"]: wd.ravel()})
    assert c["error"] == "", c["error"] + c["log"]
    log = c["log"]
    assert "[rmsnorm]" in log                                   # the RMSNorm tuner ran
    for region in ("Add + RMSNorm", "SiLU + Mul"):
        assert f"({region}): unfused kernels match the reference" in log, log
        assert log.count(f"({region}): fused at") == 3, log    # 64, 128 and 256 threads
    names = c["graph"].unit_names()
    assert any(n.startswith("Add + RMSNorm") for n in names), names
    assert any(n.startswith("SiLU + Mul") for n in names), names
    assert names.count("MatMul") == 3, names
    res = c["graph"].run()
    assert res["passed"], res["error"]
    assert res["gpu_us"] is not None and res["gpu_us"] > 0
    y = np.asarray(res["outputs"][0]).reshape(rows, hidden)
    # oracle: the reference's op composition with fp16 storage between ops
    st = lambda x: orc.store(x, F16)  # noqa: E731
    _, n = orc.add_rmsnorm(orc.f16(h), orc.f16(r), orc.f16(gamma), F16, 1e-6)
    n16 = orc.f16(st(n))
    gate = orc.f16(st(orc.linear(n16, orc.f16(wg), F16)))
    up = orc.f16(st(orc.linear(n16, orc.f16(wu), F16)))
    prod = orc.f16(st(orc.silu_mul(gate, up, F16)))
    want = orc.linear(prod, orc.f16(wd), F16)
    assert_f16_path(y, want, what=f"C2 graph rows={rows}")
    # a second run reuses the prepared units
    again = c["graph"].run()
    assert again["passed"] and np.array_equal(np.asarray(again["outputs"][0]), np.asarray(res["outputs"][0]))


def test_views_embedding_and_fp32_norm_graph(host, orc, rt):
    """Embedding -> Reshape -> fp16 graph, and an fp32 RMSNorm read back
    through a Transpose view of its result."""
    T, O = host.TensorType, host.OpType
    g = host.TensorGraph()
    vocab, width, rows = 50, 256, 6
    table = g.add_input("table", T([vocab, width], host.DType.Float16))
    tok = g.add_input("ids", T([rows], host.DType.Int32))
    e = g.add_node(O.Embedding, [table, tok])
    e2 = g.add_node(O.Reshape, [e], host.ReshapeAttributes([2, rows // 2, width]))
    flat = g.add_node(O.View, [e2], host.ReshapeAttributes([rows, width]))
    s = g.add_node(O.SiLU, [flat])
    g.outputs = [s]
    tv = normal(930, (vocab, width))
    ids = np.array([3, 49, 0, 7, 7, 12])
    c = host.compile_graph(rt, g, {table: tv.ravel(), tok: ids.astype(np.float32)})
    assert c["error"] == "", c["error"] + c["log"]
    res = c["graph"].run()
    assert res["passed"], res["error"]
    x = orc.f16_values(orc.f16(tv))[ids].astype(np.float64)
    want = x / (1.0 + np.exp(-x))
    assert_f16_path(np.asarray(res["outputs"][0]).reshape(rows, width), want, "embedding + SiLU")

    g = host.TensorGraph()
    xr = normal(931, (3, 4097))
    xr[1] *= 1e-4
    w = uniform(932, (4097,), 0.5, 1.5)
    xi = g.add_input("x", T([3, 4097], host.DType.Float32))
    wi = g.add_input("w", T([4097], host.DType.Float32))
    y = g.add_node(O.RMSNorm, [xi, wi], host.RMSNormAttributes(1e-6))
    yt = g.add_node(O.Transpose, [y], host.TransposeAttributes(0, 1))
    g.outputs = [yt]
    c = host.compile_graph(rt, g, {xi: xr.ravel(), wi: w})
    assert c["error"] == "", c["error"] + c["log"]
    res = c["graph"].run()
    assert res["passed"], res["error"]
    want = orc.rmsnorm(xr, w, F32, 1e-6)
    assert_f32_rel(np.asarray(res["outputs"][0]).reshape(4097, 3), want.T, what="fp32 RMSNorm^T")


def test_compile_errors_name_the_cause(host, rt):
    T, O = host.TensorType, host.OpType
    g = host.TensorGraph()
    x = g.add_input("x", T([1, 64], host.DType.Float16))
    w = g.add_input("w", T([64, 32], host.DType.Float16))   # [K, N], not a Transpose view
    g.outputs = [g.add_node(O.MatMul, [x, w])]
    c = host.compile_graph(rt, g, {x: np.zeros(64, np.float32), w: np.zeros(64 * 32, np.float32)})
    assert c["graph"] is None and "nn.Linear layout" in c["error"]
    g = host.TensorGraph()
    x = g.add_input("x", T([4, 8], host.DType.Float16))
    g.outputs = [g.add_node(O.ReLU, [x])]
    c = host.compile_graph(rt, g, {x: np.zeros(32, np.float32)})
    assert c["graph"] is None and "ReLU is not in the gfx950 graph path's op set" in c["error"]
    g = host.TensorGraph()
    x = g.add_input("x", T([4, 8], host.DType.Float16))
    g.outputs = [g.add_node(O.SiLU, [x])]
    c = host.compile_graph(rt, g, {x: np.zeros(5, np.float32)})
    assert c["graph"] is None and "needs 32 host values" in c["error"]
