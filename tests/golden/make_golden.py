"""Write tests/golden/golden.npz from the reference's own CPU oracle.

Runs in the build container only (it needs /root/reference): builds
oracle/_ref/libtmc_ref.so from the reference sources (oracle/Makefile,
target ``ref``), evaluates small TensorIR graphs with the reference
``evaluateGraph`` (GraphReference.cpp:98-339) and ``compare``
(Validator.cpp:11-38), and stores inputs and outputs as plain arrays.
The fixtures pin oracle/tmc_oracle.c (tests/test_oracle.py).

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libtmc_ref.so")
OUT = os.path.join(HERE, "golden.npz")

F16, F32, BF16, I32 = 0, 1, 2, 3


def graph_data(count: int, seed: int = 0, scale: float = 1.0) -> np.ndarray:
    """Deterministic inputs of tensor_graph_examples.cpp:18-25."""
    i = np.arange(count, dtype=np.int64)
    centered = ((i * 17 + seed * 13) % 257) - 128
    return (centered.astype(np.float32) / np.float32(64.0)) * np.float32(scale)


def f16_ties() -> np.ndarray:
    """fp32 values that sit exactly halfway between adjacent fp16 values,
    plus boundary cases (subnormal ties, overflow edge, specials)."""
    rng = np.random.default_rng(7)
    halves = rng.integers(0, 0x7bff, size=96, dtype=np.uint16)
    lo = halves.view(np.float16).astype(np.float64)
    hi = (halves + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)  # exact in fp32
    specials = np.array([0.0, -0.0, 1.0, -1.0, 1.0 + 2.0 ** -11, -(1.0 + 2.0 ** -11),
                         1.0 + 3 * 2.0 ** -11, 2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -26,
                         2.0 ** -24, 1.5 * 2.0 ** -24, 6.1e-5, 65504.0, 65519.0, 65520.0,
                         65536.0, 1e6, -1e6, np.inf, -np.inf, np.nan, 1e-8, -1e-8,
                         2.0 ** -14, 2.0 ** -14 - 2.0 ** -25],
                        dtype=np.float32)
    normal = rng.standard_normal(64).astype(np.float32)
    small = (rng.standard_normal(64) * 0.02).astype(np.float32)
    tiny = (rng.standard_normal(64) * 1e-5).astype(np.float32)
    return np.concatenate([mids, -mids, specials, normal, small, tiny]).astype(np.float32)


class Ref:
    def __init__(self):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True)
        self.l = C.CDLL(REF_LIB)
        self.l.ref_last_error.restype = C.c_char_p

    def _ok(self, rc):
        if rc != 0:
            raise RuntimeError(self.l.ref_last_error().decode())

    @staticmethod
    def p(a):
        return a.ctypes.data_as(C.c_void_p)

    def store(self, x, dtype):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self._ok(self.l.ref_store(self.p(x), C.c_size_t(x.size), dtype, self.p(out)))
        return out

    def rmsnorm(self, x, w, dtype, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty(x.shape, np.float64)
        self._ok(self.l.ref_rmsnorm(self.p(x), self.p(w), C.c_size_t(x.shape[0]),
                                    C.c_size_t(x.shape[1]), dtype, C.c_float(eps), self.p(out)))
        return out

    def add_rmsnorm(self, x, r, w, dtype, eps):
        x = np.ascontiguousarray(x, np.float32)
        r = np.ascontiguousarray(r, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        s = np.empty(x.shape, np.float32)
        out = np.empty(x.shape, np.float64)
        self._ok(self.l.ref_add_rmsnorm(self.p(x), self.p(r), self.p(w), C.c_size_t(x.shape[0]),
                                        C.c_size_t(x.shape[1]), dtype, C.c_float(eps),
                                        self.p(s), self.p(out)))
        return s, out

    def matmul(self, a, b, dtype):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        out = np.empty((a.shape[0], b.shape[1]), np.float64)
        self._ok(self.l.ref_matmul(self.p(a), self.p(b), C.c_size_t(a.shape[0]),
                                   C.c_size_t(a.shape[1]), C.c_size_t(b.shape[1]), dtype,
                                   self.p(out)))
        return out

    def silu_mul(self, g, u, dtype):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        out = np.empty(g.shape, np.float64)
        self._ok(self.l.ref_silu_mul(self.p(g), self.p(u), C.c_size_t(g.size), dtype, self.p(out)))
        return out

    def rope(self, x, cos, sin, rows, heads, d):
        x = np.ascontiguousarray(x, np.float32)
        cos = np.ascontiguousarray(cos, np.float32)
        sin = np.ascontiguousarray(sin, np.float32)
        out = np.empty(x.size, np.float64)
        self._ok(self.l.ref_rope(self.p(x), self.p(cos), self.p(sin), C.c_size_t(rows),
                                 C.c_size_t(heads), C.c_size_t(d), self.p(out)))
        return out

    def attention(self, q, k, v, pairs, length, d, scale):
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        out = np.empty(pairs * d, np.float64)
        self._ok(self.l.ref_attention(self.p(q), self.p(k), self.p(v), C.c_size_t(pairs),
                                      C.c_size_t(length), C.c_size_t(d), C.c_float(scale),
                                      self.p(out)))
        return out

    def gather_rows(self, table, idx):
        table = np.ascontiguousarray(table, np.float32)
        idx = np.ascontiguousarray(idx, np.float32)
        out = np.empty((idx.size, table.shape[1]), np.float64)
        self._ok(self.l.ref_gather_rows(self.p(table), C.c_size_t(table.shape[0]),
                                        C.c_size_t(table.shape[1]), self.p(idx),
                                        C.c_size_t(idx.size), self.p(out)))
        return out

    def compare(self, actual, ref, atol, rtol):
        a = np.ascontiguousarray(actual, np.float32)
        r = np.ascontiguousarray(ref, np.float64)
        worst, mism = C.c_double(), C.c_size_t()
        self.l.ref_compare.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_double,
                                       C.c_double, C.POINTER(C.c_double),
                                       C.POINTER(C.c_size_t)]
        ok = self.l.ref_compare(self.p(a), self.p(r), a.size, atol, rtol, C.byref(worst),
                                C.byref(mism))
        return np.array([ok, worst.value, mism.value], np.float64)


def main() -> None:
    ref = Ref()
    g = {}
    rng = np.random.default_rng(2024)

    # storage rounding
    ties = f16_ties()
    g["store_in"] = ties
    g["store_f16"] = ref.store(ties, F16)
    g["store_f32"] = ref.store(ties, F32)
    g["store_bf16"] = ref.store(ties, BF16)
    ints = np.array([0.0, 0.9, -0.9, 1.5, -1.5, 2.7, -2.7, 1e6 + 0.5, -3e5 - 0.75, 7.0],
                    np.float32)
    g["store_i32_in"] = ints
    g["store_i32"] = ref.store(ints, I32)

    # RMSNorm cases of tensor_graph_examples.cpp:89-99,247-250
    def rms_inputs(rows, width):
        x = graph_data(rows * width).reshape(rows, width)
        if rows > 1:
            x[0, :] = 0.0
            x[1, :] *= np.float32(1e-4)
        w = (np.float32(0.5) + (np.arange(width) % 31).astype(np.float32) / np.float32(32.0))
        return x.astype(np.float32), w.astype(np.float32)

    for name, rows, width, dtype, eps in (("rms_1x4096", 1, 4096, F32, 1e-5),
                                          ("rms_3x4097", 3, 4097, F32, 1e-5),
                                          ("rms_3x4097_e6", 3, 4097, F32, 1e-6),
                                          ("rms_f16_1x257", 1, 257, F16, 1e-5),
                                          ("rms_f16_4x512", 4, 512, F16, 1e-6)):
        x, w = rms_inputs(rows, width)
        if name == "rms_f16_4x512":
            x = rng.standard_normal((rows, width)).astype(np.float32)
            w = rng.uniform(0.5, 1.5, width).astype(np.float32)
        g[f"{name}_x"], g[f"{name}_w"] = x, w
        g[f"{name}_meta"] = np.array([dtype, eps], np.float64)
        g[f"{name}_out"] = ref.rmsnorm(x, w, dtype, eps)

    for name, rows, width, dtype in (("addrms_3x4097", 3, 4097, F32),
                                     ("addrms_f16_2x257", 2, 257, F16),
                                     ("addrms_f16_3x4096", 3, 4096, F16)):
        x, w = rms_inputs(rows, width)
        r = (rng.standard_normal((rows, width)) * (0.1 if dtype == F32 else 1.0)).astype(
            np.float32)
        if dtype == F16:
            x = rng.standard_normal((rows, width)).astype(np.float32)
        s, out = ref.add_rmsnorm(x, r, w, dtype, 1e-6)
        g[f"{name}_x"], g[f"{name}_r"], g[f"{name}_w"] = x, r, w
        g[f"{name}_dtype"] = np.array([dtype], np.int64)
        g[f"{name}_sum"], g[f"{name}_out"] = s, out

    # MatMul: graph example shape and an fp16 linear-like shape (W^T operand)
    a = graph_data(21).reshape(3, 7)
    b = graph_data(35, 1, 0.25).reshape(7, 5)
    g["mm_f32_a"], g["mm_f32_b"], g["mm_f32_out"] = a, b, ref.matmul(a, b, F32)
    x = rng.standard_normal((2, 64)).astype(np.float32)
    wt = (rng.standard_normal((64, 48)) * 0.02).astype(np.float32)
    g["mm_f16_a"], g["mm_f16_b"], g["mm_f16_out"] = x, wt, ref.matmul(x, wt, F16)

    # SiLU -> Mul (sign-stable SiLU, GraphReference.cpp:143-149)
    for name, n, dtype in (("silu_f32", 51, F32), ("silu_f16", 257, F16)):
        gate = (rng.standard_normal(n) * 4).astype(np.float32)
        gate[:6] = [20.0, -20.0, 100.0, -100.0, 0.0, -1e-3]
        up = rng.standard_normal(n).astype(np.float32)
        g[f"{name}_g"], g[f"{name}_u"] = gate, up
        g[f"{name}_out"] = ref.silu_mul(gate, up, dtype)

    # RoPE interleaved pairs with per-row tables
    rows, heads, d = 3, 2, 8
    xr = graph_data(rows * heads * d)
    pos = np.arange(rows)
    ang = pos[:, None] / np.power(10000.0, np.arange(d // 2)[None, :] / (d // 2))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    g["rope_x"], g["rope_cos"], g["rope_sin"] = xr, cos, sin
    g["rope_out"] = ref.rope(xr, cos, sin, rows, heads, d)

    # attention chain MatMul -> Mul(scale) -> Softmax -> MatMul
    pairs, length, d = 3, 17, 16
    q = rng.standard_normal((pairs, 1, d)).astype(np.float32)
    k = rng.standard_normal((pairs, length, d)).astype(np.float32)
    v = rng.standard_normal((pairs, length, d)).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(d))
    g["attn_q"], g["attn_k"], g["attn_v"] = q, k, v
    g["attn_meta"] = np.array([pairs, length, d, scale], np.float64)
    g["attn_out"] = ref.attention(q, k, v, pairs, length, d, float(scale))

    # Gather of pages (block-table walk) along axis 0
    table = graph_data(6 * 10, 5).reshape(6, 10)
    idx = np.array([4, 0, 5, 2], np.float32)
    g["gather_table"], g["gather_idx"], g["gather_out"] = table, idx, ref.gather_rows(table, idx)

    # Validator::compare
    actual = np.array([1.0, 2.0, 3.5, np.nan, 4.0], np.float32)
    expected = np.array([1.0, 2.001, 3.0, 1.0, 4.0 + 1e-4], np.float64)
    g["cmp_actual"], g["cmp_ref"] = actual, expected
    g["cmp_out_a"] = ref.compare(actual[:3], expected[:3], 1e-3, 1e-3)
    g["cmp_out_b"] = ref.compare(actual, expected, 1e-3, 1e-3)
    g["cmp_out_c"] = ref.compare(actual[[0, 1, 4]], expected[[0, 1, 4]], 2e-3, 0.0)

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} with {len(g)} arrays")


if __name__ == "__main__":
    main()
