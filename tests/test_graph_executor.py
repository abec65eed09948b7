"""The graph path's host logic (no GPU): TensorIR type inference and views,
fusion-region formation and the product-side graph reference, the last
checked against the pinned oracle (GraphExecutor.cpp:346-430,
PatternAnalyzer.cpp:34-131, GraphAnalyzer.cpp, GraphReference.cpp)."""
import numpy as np
import pytest

from tests.helpers import F16, F32, normal, uniform


def _mlp_graph(host, rows, hidden, inter, dtype):
    """C2's block as TensorIR: Add -> RMSNorm -> gate/up MatMuls (weights as
    Transpose views of [N, K] tensors) -> SiLU -> Mul -> down MatMul."""
    T = host.TensorType
    g = host.TensorGraph()
    h = g.add_input("h", T([rows, hidden], dtype))
    r = g.add_input("r", T([rows, hidden], dtype))
    gamma = g.add_input("gamma", T([hidden], dtype))
    wg = g.add_input("wg", T([inter, hidden], dtype))
    wu = g.add_input("wu", T([inter, hidden], dtype))
    wd = g.add_input("wd", T([hidden, inter], dtype))
    O = host.OpType
    s = g.add_node(O.Add, [h, r], None, "s")
    n = g.add_node(O.RMSNorm, [s, gamma], host.RMSNormAttributes(1e-6), "n")
    wgt = g.add_node(O.Transpose, [wg], host.TransposeAttributes(0, 1), "wg_t")
    wut = g.add_node(O.Transpose, [wu], host.TransposeAttributes(0, 1), "wu_t")
    wdt = g.add_node(O.Transpose, [wd], host.TransposeAttributes(0, 1), "wd_t")
    gate = g.add_node(O.MatMul, [n, wgt], None, "gate")
    up = g.add_node(O.MatMul, [n, wut], None, "up")
    act = g.add_node(O.SiLU, [gate], None, "act")
    prod = g.add_node(O.Mul, [act, up], None, "prod")
    y = g.add_node(O.MatMul, [prod, wdt], None, "y")
    g.outputs = [y]
    return g, dict(h=h, r=r, gamma=gamma, wg=wg, wu=wu, wd=wd, y=y, n=n, prod=prod)


def test_types_views_and_aliases(host):
    g, ids = _mlp_graph(host, 2, 64, 96, host.DType.Float16)
    a = host.analyze_graph(g)
    types = a["types"]
    wgt = types[ids["wg"] + 0]  # the weight itself: contiguous [96, 64]
    assert list(wgt.shape) == [96, 64] and wgt.is_contiguous()
    # the Transpose views: [64, 96], strides (1, 64), aliasing their weight
    views = [v for v, base in enumerate(a["alias_of"]) if base is not None]
    assert len(views) == 3
    for v in views:
        t = types[v]
        assert not t.is_contiguous() and t.layout == host.Layout.Strided
        assert list(t.strides()) == [1, t.shape[0]]
        assert t.storage_element_count() == t.element_count()
    assert list(types[ids["y"]].shape) == [2, 64]


def test_analysis_rejects_what_the_kernels_cannot_run(host):
    T, O = host.TensorType, host.OpType
    g = host.TensorGraph()
    x = g.add_input("x", T([4, 8], host.DType.Float16))
    g.add_node(O.Softmax, [x], host.SoftmaxAttributes(-1))
    with pytest.raises(Exception, match="Softmax is not in the gfx950 graph path's op set"):
        host.analyze_graph(g)
    g = host.TensorGraph()
    x = g.add_input("x", T([4, 8], host.DType.Float16))
    y = g.add_input("y", T([1, 8], host.DType.Float16))
    g.add_node(O.Add, [x, y])
    with pytest.raises(Exception, match="no broadcasting"):
        host.analyze_graph(g)
    g = host.TensorGraph()
    x = g.add_input("x", T([4, 8], host.DType.Float16))
    g.add_node(O.Reshape, [x], host.ReshapeAttributes([5, 7]))
    with pytest.raises(Exception, match="equal element counts"):
        host.analyze_graph(g)
    g = host.TensorGraph()
    x = g.add_input("x", T([4, 8], host.DType.Float16))
    w = g.add_input("w", T([9, 8], host.DType.Float16))
    g.add_node(O.MatMul, [x, w])
    with pytest.raises(Exception, match=r"\[M, K\] x \[K, N\]"):
        host.analyze_graph(g)


def test_regions_follow_exclusive_contiguous_edges(host):
    g, ids = _mlp_graph(host, 2, 64, 96, host.DType.Float16)
    regions = host.graph_regions(g)
    fused = [r["fusion"] for r in regions if r["fusion"] != "Unfused"]
    assert fused == ["Add + RMSNorm", "SiLU + Mul"]
    add_norm = next(r for r in regions if r["fusion"] == "Add + RMSNorm")
    assert add_norm["outputs"] == [ids["n"]]               # the sum stays inside
    assert set(add_norm["inputs"]) == {ids["h"], ids["r"], ids["gamma"]}
    silu_mul = next(r for r in regions if r["fusion"] == "SiLU + Mul")
    assert silu_mul["outputs"] == [ids["prod"]]
    # the sum also read elsewhere (a graph output): no fusion
    g2, ids2 = _mlp_graph(host, 2, 64, 96, host.DType.Float16)
    g2.outputs = [ids2["y"], ids2["n"] - 1]  # the Add's result
    assert "Add + RMSNorm" not in [r["fusion"] for r in host.graph_regions(g2)]
    # SiLU read by two nodes: no fusion
    T, O = host.TensorType, host.OpType
    g3 = host.TensorGraph()
    a = g3.add_input("a", T([8], host.DType.Float16))
    b = g3.add_input("b", T([8], host.DType.Float16))
    s = g3.add_node(O.SiLU, [a])
    m1 = g3.add_node(O.Mul, [s, b])
    m2 = g3.add_node(O.Mul, [s, a])
    g3.outputs = [m1, m2]
    assert all(r["fusion"] == "Unfused" for r in host.graph_regions(g3))


def test_graph_reference_matches_the_oracle(host, orc):
    """The product's graph reference (every stored value rounded to its
    dtype) against the pinned oracle's ops on the C2 structure."""
    rows, hidden, inter = 3, 64, 96
    odt = F16
    g, ids = _mlp_graph(host, rows, hidden, inter, host.DType.Float16)
    h = normal(901, (rows, hidden))
    r = normal(902, (rows, hidden))
    gamma = uniform(903, (hidden,), 0.5, 1.5)
    wg, wu = normal(904, (inter, hidden), 0.1), normal(905, (inter, hidden), 0.1)
    wd = normal(906, (hidden, inter), 0.1)
    inputs = {ids["h"]: h.ravel(), ids["r"]: r.ravel(), ids["gamma"]: gamma,
              ids["wg"]: wg.ravel(), ids["wu"]: wu.ravel(), ids["wd"]: wd.ravel()}
    ref = host.evaluate_graph(g, {k: list(map(float, v)) for k, v in inputs.items()})
    st = lambda x: orc.store(x, odt)  # noqa: E731
    h16, r16, g16 = orc.f16(h), orc.f16(r), orc.f16(gamma)
    s, n = orc.add_rmsnorm(h16, r16, g16, odt, 1e-6)
    n = st(n)
    gate, up = st(orc.linear(orc.f16(n), orc.f16(wg), odt)), st(orc.linear(orc.f16(n), orc.f16(wu), odt))
    prod = st(orc.silu_mul(orc.f16(gate), orc.f16(up), odt))
    y = st(orc.linear(orc.f16(prod), orc.f16(wd), odt))
    got = np.asarray(ref["values"][ids["n"]]).reshape(rows, hidden)
    np.testing.assert_array_equal(got, n)
    np.testing.assert_array_equal(np.asarray(ref["values"][ids["prod"]]).reshape(rows, inter), prod)
    np.testing.assert_array_equal(np.asarray(ref["outputs"][0]).reshape(rows, hidden), y)


def test_graph_reference_rmsnorm_fp32_and_views(host, orc):
    T, O = host.TensorType, host.OpType
    rows, width = 3, 4097
    x = normal(911, (rows, width))
    x[0] = 0.0
    x[1] *= 1e-4
    w = uniform(912, (width,), 0.5, 1.5)
    g = host.TensorGraph()
    xi = g.add_input("x", T([rows * width], host.DType.Float32))
    wi = g.add_input("w", T([width], host.DType.Float32))
    xr = g.add_node(O.Reshape, [xi], host.ReshapeAttributes([rows, width]))
    y = g.add_node(O.RMSNorm, [xr, wi], host.RMSNormAttributes(1e-6))
    yt = g.add_node(O.Transpose, [y], host.TransposeAttributes(0, 1))
    g.outputs = [y, yt]
    ref = host.evaluate_graph(g, {xi: list(map(float, x.ravel())), wi: list(map(float, w))})
    want = orc.store(orc.rmsnorm(x, w, F32, 1e-6), F32)
    np.testing.assert_array_equal(np.asarray(ref["outputs"][0]).reshape(rows, width), want)
    np.testing.assert_array_equal(np.asarray(ref["outputs"][1]).reshape(width, rows), want.T)


def test_graph_reference_embedding_bounds(host):
    T, O = host.TensorType, host.OpType
    g = host.TensorGraph()
    table = g.add_input("table", T([5, 4], host.DType.Float16))
    ids = g.add_input("ids", T([3], host.DType.Int32))
    e = g.add_node(O.Embedding, [table, ids])
    g.outputs = [e]
    tv = [float(i) for i in range(20)]
    ref = host.evaluate_graph(g, {table: tv, ids: [4.0, 0.0, 2.0]})
    assert ref["outputs"][0] == tv[16:20] + tv[0:4] + tv[8:12]
    with pytest.raises(Exception, match="Embedding index is out of range"):
        host.evaluate_graph(g, {table: tv, ids: [5.0, 0.0, 0.0]})
