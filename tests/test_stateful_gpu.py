"""GPU: the KV-cache attention module executor (compileKVCacheAttention,
reference src/runtime/StatefulExecutor.cpp:134-265; the KVCache.py module
MultiHeadAttentionKVCache with no mask) against the oracle on the same fp16
inputs: projections (double sums, stored fp16), the K/V cache append, the
attention of every query over every cached position (stored fp16) and the o
projection.  Includes C3's shape (32 heads x 128, capacity 4096): the cache
filled to L = 4095 by a prefill, one decode to 4096, and the next decode
rejected with "KV cache capacity has been reached." and the state unchanged
(StatefulExecutor.cpp:196-207).

Tolerances: outputs and cache contents are fp16-path values (2e-2 absolute,
3e-3 relative RMS); a rejected call leaves the cache bit-identical."""
import os

import numpy as np
import pytest

from tests.helpers import assert_f16_path

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt(host):
    r = host.HipRuntime()
    assert r.is_available(), r.initialization_error()
    return r


class ModuleOracle:
    """The module on the oracle, every stored tensor fp16: the caches are
    [batch][heads][capacity][head_dim] bits, used as one page per batch."""

    def __init__(self, orc, batch, heads, d, capacity, weights):
        self.orc, self.B, self.H, self.D, self.cap = orc, batch, heads, d, capacity
        self.wq, self.wk, self.wv, self.wo = weights
        self.k = np.zeros((batch, heads, capacity, d), np.uint16)
        self.v = np.zeros_like(self.k)
        self.length = 0

    def project(self, x_bits, w, rows=None):
        x = x_bits if rows is None else x_bits[rows]
        return self.orc.f16(self.orc.linear_values(x, w).astype(np.float32))

    def step(self, xq, xk, xv, rows=None):
        """One call of S = len(xq) / batch rows; returns the fp16 output bits
        of `rows` (all by default)."""
        orc, B, H, D = self.orc, self.B, self.H, self.D
        S = xq.shape[0] // B
        for x, cache in ((xk, self.k), (xv, self.v)):
            p = self.project(x, self.wk if cache is self.k else self.wv).reshape(B, S, H, D)
            cache[:, :, self.length:self.length + S, :] = p.transpose(0, 2, 1, 3)
        self.length += S
        picked = np.arange(B * S) if rows is None else np.asarray(rows)
        q = self.project(xq, self.wq, picked)
        ctx, written = orc.paged_attention(
            q, self.k.ravel(), self.v.ravel(), orc.F16, H, H, D, self.cap, H * self.cap * D,
            self.cap * D, (picked // S)[:, None], 1, np.full(picked.size, self.length), picked.size)
        assert written.all()
        return self.project(orc.f16(ctx.astype(np.float32)), self.wo)


def _plan(host, batch, heads, d, capacity, prefill):
    plan = host.KVCachePlan()
    plan.batch, plan.heads, plan.head_dimension = batch, heads, d
    plan.capacity, plan.prefill_length = capacity, prefill
    plan.threads_per_threadgroup = max(128, d)
    plan.dtype = host.DType.Float16
    return plan


def _weights(orc, rng, dim):
    bound = 1.0 / np.sqrt(dim)
    return [orc.f16(rng.uniform(-bound, bound, (dim, dim)).astype(np.float32)) for _ in range(4)]


def _inputs(orc, rng, rows, dim):
    return [orc.f16(rng.standard_normal((rows, dim), dtype=np.float32)) for _ in range(3)]


@pytest.mark.parametrize("batch,heads,d,capacity,prefill", [(1, 4, 64, 24, 9), (2, 2, 128, 20, 17),
                                                            (1, 8, 16, 12, 3)])
def test_kv_module_matches_oracle_to_capacity(host, orc, rt, batch, heads, d, capacity, prefill):
    rng = np.random.default_rng(900 + heads)
    dim = heads * d
    w = _weights(orc, rng, dim)
    vals = orc.f16_values
    exe, log = host.compile_kv_cache_attention(rt, _plan(host, batch, heads, d, capacity, prefill),
                                               *[vals(x).ravel() for x in w])
    assert "KV attention module compiled" in log
    ref = ModuleOracle(orc, batch, heads, d, capacity, w)
    bad = exe.decode(*[np.zeros(batch * dim, np.float32)] * 3)
    assert not bad["passed"] and bad["error"] == "Decode requires a completed prefill."
    xs = _inputs(orc, rng, batch * prefill, dim)
    out = exe.prefill(*[vals(x).ravel() for x in xs])
    assert out["passed"], out["error"]
    assert_f16_path(out["output"], vals(ref.step(*xs)), "prefill output")
    again = exe.prefill(*[vals(x).ravel() for x in xs])
    assert not again["passed"] and "call reset first" in again["error"]
    for step in range(capacity - prefill):
        xs = _inputs(orc, rng, batch, dim)
        out = exe.decode(*[vals(x).ravel() for x in xs])
        assert out["passed"], out["error"]
        assert_f16_path(out["output"], vals(ref.step(*xs)), f"decode {step} output")
    assert exe.current_length() == capacity
    assert_f16_path(exe.read_key_prefix(), vals(ref.k), "key cache")
    assert_f16_path(exe.read_value_prefix(), vals(ref.v), "value cache")
    keys, values = exe.read_key_prefix(), exe.read_value_prefix()
    full = exe.decode(*[vals(x).ravel() for x in _inputs(orc, rng, batch, dim)])
    assert not full["passed"] and full["error"] == "KV cache capacity has been reached."
    assert exe.current_length() == capacity
    assert np.array_equal(exe.read_key_prefix(), keys)
    assert np.array_equal(exe.read_value_prefix(), values)
    short = exe.reset()
    assert short == "" and exe.current_length() == 0
    wrong = exe.prefill(*[np.zeros(3, np.float32)] * 3)
    assert not wrong["passed"] and "input shape" in wrong["error"]


def test_c3_shape_fills_capacity_then_rejects(host, orc, rt):
    """C3: 32 heads x 128, fixed capacity 4096, a prefill of L = 4095
    tokens, the decode that appends at position 4095, then rejection."""
    batch, heads, d, capacity, L = 1, 32, 128, 4096, 4095
    dim = heads * d
    rng = np.random.default_rng(3300)
    w = _weights(orc, rng, dim)
    vals = orc.f16_values
    exe, _ = host.compile_kv_cache_attention(rt, _plan(host, batch, heads, d, capacity, L),
                                             *[vals(x).ravel() for x in w])
    xs = _inputs(orc, rng, L, dim)
    print("[c3] prefill of 4095 tokens", flush=True)
    out = exe.prefill(*[vals(x).ravel() for x in xs])
    assert out["passed"], out["error"]
    orc.set_threads(max(1, min(16, os.cpu_count() or 1)))
    try:
        ref = ModuleOracle(orc, batch, heads, d, capacity, w)
        sample = np.array([0, 1, 17, 511, 2048, 3000, 4093, 4094])
        want = ref.step(*xs, rows=sample)
        print("[c3] oracle prefill done", flush=True)
        got = out["output"].reshape(L, dim)[sample]
        assert_f16_path(got, vals(want), "prefill output (sampled rows)")
        assert_f16_path(exe.read_key_prefix(), vals(ref.k[:, :, :L]), "key cache after prefill")
        xs = _inputs(orc, rng, 1, dim)
        out = exe.decode(*[vals(x).ravel() for x in xs])
        assert out["passed"], out["error"]
        assert_f16_path(out["output"], vals(ref.step(*xs)), "decode at position 4095")
    finally:
        orc.set_threads(1)
    assert exe.current_length() == capacity
    keys, values = exe.read_key_prefix(), exe.read_value_prefix()
    assert_f16_path(values, vals(ref.v), "value cache at capacity")
    full = exe.decode(*[vals(x).ravel() for x in _inputs(orc, rng, 1, dim)])
    assert not full["passed"] and full["error"] == "KV cache capacity has been reached."
    assert exe.current_length() == capacity
    assert np.array_equal(exe.read_key_prefix(), keys)
    assert np.array_equal(exe.read_value_prefix(), values)
