"""numpy front end of the CPU oracle (oracle/libtmc_oracle.so).

TEST INFRASTRUCTURE ONLY: used by tests/, ``__graft_entry__.smoke()`` and
bench.py's cpu_baseline leg as the checker; the product library never loads
it.  Each wrapper names the C function it calls; the C file cites the
reference file:line each function restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtmc_oracle.so")

F16, F32, BF16, I32 = 0, 1, 2, 3
_NP = {F16: np.uint16, F32: np.float32, BF16: np.uint16, I32: np.int32}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _declare(l):
    vp, sz, dp, fp = C.c_void_p, C.c_size_t, C.c_double, C.c_float
    l.tmco_f32_to_f16.restype = C.c_uint16
    l.tmco_f32_to_f16.argtypes = [fp]
    l.tmco_f16_to_f32.restype = fp
    l.tmco_f16_to_f32.argtypes = [C.c_uint16]
    l.tmco_store.restype = fp
    l.tmco_store.argtypes = [dp, C.c_int]
    l.tmco_encode.argtypes = [vp, sz, C.c_int, vp]
    l.tmco_decode.argtypes = [vp, sz, C.c_int, vp]
    l.tmco_compare.restype = C.c_int
    l.tmco_compare.argtypes = [vp, vp, sz, dp, dp, C.POINTER(dp), C.POINTER(sz), C.POINTER(sz)]
    l.tmco_rmsnorm_reference.argtypes = [vp, vp, sz, sz, fp, vp]
    l.tmco_rmsnorm.argtypes = [vp, vp, C.c_int, sz, sz, fp, vp]
    l.tmco_add_rmsnorm.argtypes = [vp, vp, vp, C.c_int, sz, sz, fp, vp, vp]
    l.tmco_linear.argtypes = [vp, vp, C.c_int, sz, sz, sz, vp]
    l.tmco_silu_mul.argtypes = [vp, vp, C.c_int, sz, vp]
    l.tmco_gated_mlp.argtypes = [vp, vp, vp, C.c_int, sz, sz, sz, vp]
    l.tmco_rope.argtypes = [vp, vp, vp, C.c_int, sz, sz, sz, vp, vp]
    l.tmco_decode_attention.argtypes = [vp, vp, vp, C.c_int, sz, sz, sz, sz, sz, sz, vp]
    l.tmco_paged_attention.restype = C.c_int
    l.tmco_paged_attention.argtypes = [vp, vp, vp, C.c_int, sz, sz, sz, sz, sz, sz, sz, vp, sz,
                                       vp, sz, vp, vp]
    l.tmco_argmax.argtypes = [vp, sz, sz, vp]
    l.tmco_append_contiguous.argtypes = [vp, sz, sz, sz, sz, sz, C.c_int, C.c_int32, vp]
    l.tmco_append_paged.argtypes = [vp, sz, sz, sz, sz, sz, sz, C.c_int, C.c_int32, vp, vp]
    l.tmco_append_serving.argtypes = [vp, sz, sz, sz, sz, sz, C.c_int, vp, vp, C.c_int32, vp]
    l.tmco_set_threads.argtypes = [C.c_int]
    l.tmco_linear_values.argtypes = [vp, vp, sz, sz, sz, vp]
    l.tmco_decoder_step.restype = C.c_int
    l.tmco_decoder_step.argtypes = [vp, vp, vp, sz, sz, vp, vp, vp, sz, sz, sz, vp, vp]


# ---------------------------------------------------------------- conversions
def encode(values, dtype: int) -> np.ndarray:
    """Host upload conversion (tmco_encode): fp32 -> storage bits."""
    src = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(src.shape, dtype=_NP[dtype])
    lib().tmco_encode(_p(src), src.size, dtype, _p(out))
    return out


def decode(bits, dtype: int) -> np.ndarray:
    src = np.ascontiguousarray(bits, dtype=_NP[dtype])
    out = np.empty(src.shape, dtype=np.float32)
    lib().tmco_decode(_p(src), src.size, dtype, _p(out))
    return out


def f16(values) -> np.ndarray:
    """fp32 -> fp16 bits with the reference host rule (ties away from zero)."""
    return encode(values, F16)


def f16_values(bits) -> np.ndarray:
    return decode(bits, F16)


def store(values, dtype: int) -> np.ndarray:
    """storeValue of each element (tmco_store)."""
    src = np.ascontiguousarray(values, dtype=np.float64).ravel()
    f = lib().tmco_store
    return np.array([f(float(v), dtype) for v in src], dtype=np.float32).reshape(np.shape(values))


# ---------------------------------------------------------------- validator
def compare(actual, reference, atol: float, rtol: float):
    a = np.ascontiguousarray(actual, dtype=np.float32).ravel()
    r = np.ascontiguousarray(reference, dtype=np.float64).ravel()
    worst, mism, first = C.c_double(), C.c_size_t(), C.c_size_t()
    ok = lib().tmco_compare(_p(a), _p(r), a.size, atol, rtol, C.byref(worst), C.byref(mism),
                            C.byref(first))
    return bool(ok), worst.value, mism.value


def rmsnorm_reference(x, w, epsilon: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, width = x.shape
    out = np.empty((rows, width), dtype=np.float64)
    lib().tmco_rmsnorm_reference(_p(x), _p(w), rows, width, epsilon, _p(out))
    return out


# ---------------------------------------------------------------- ops
def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=_NP[dtype])


def rmsnorm(x, w, dtype: int, epsilon: float) -> np.ndarray:
    x, w = _c(x, dtype), _c(w, dtype)
    rows, width = x.shape
    out = np.empty((rows, width), dtype=np.float64)
    lib().tmco_rmsnorm(_p(x), _p(w), dtype, rows, width, epsilon, _p(out))
    return out


def add_rmsnorm(residual, update, w, dtype: int, epsilon: float):
    r, u, w = _c(residual, dtype), _c(update, dtype), _c(w, dtype)
    rows, width = r.shape
    s = np.empty((rows, width), dtype=np.float32)
    out = np.empty((rows, width), dtype=np.float64)
    lib().tmco_add_rmsnorm(_p(r), _p(u), _p(w), dtype, rows, width, epsilon, _p(s), _p(out))
    return s, out


def linear(x, weight, dtype: int) -> np.ndarray:
    """y = x @ W^T, W stored [out, in]."""
    x, weight = _c(x, dtype), _c(weight, dtype)
    rows, k = x.shape
    n = weight.shape[0]
    assert weight.shape[1] == k
    y = np.empty((rows, n), dtype=np.float64)
    lib().tmco_linear(_p(x), _p(weight), dtype, rows, k, n, _p(y))
    return y


def silu_mul(gate, up, dtype: int) -> np.ndarray:
    g, u = _c(gate, dtype), _c(up, dtype)
    out = np.empty(g.shape, dtype=np.float64)
    lib().tmco_silu_mul(_p(g), _p(u), dtype, g.size, _p(out))
    return out


def gated_mlp(x, wg, wu, dtype: int) -> np.ndarray:
    x, wg, wu = _c(x, dtype), _c(wg, dtype), _c(wu, dtype)
    rows, hidden = x.shape
    inter = wg.shape[0]
    out = np.empty((rows, inter), dtype=np.float64)
    lib().tmco_gated_mlp(_p(x), _p(wg), _p(wu), dtype, rows, hidden, inter, _p(out))
    return out


def rope(x, cos, sin, dtype: int, heads: int, head_dim: int, positions) -> np.ndarray:
    x = _c(x, dtype)
    rows = x.size // (heads * head_dim)
    cos = np.ascontiguousarray(cos, dtype=np.float32)
    sin = np.ascontiguousarray(sin, dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    out = np.empty(x.size, dtype=np.float64)
    lib().tmco_rope(_p(x), _p(cos), _p(sin), dtype, rows, heads, head_dim, _p(pos), _p(out))
    return out.reshape(x.shape)


def decode_attention(q, k_cache, v_cache, dtype: int, q_heads: int, kv_heads: int, head_dim: int,
                     capacity: int, valid: int) -> np.ndarray:
    q, k_cache, v_cache = _c(q, dtype), _c(k_cache, dtype), _c(v_cache, dtype)
    batch = q.size // (q_heads * head_dim)
    out = np.empty((batch, q_heads * head_dim), dtype=np.float64)
    lib().tmco_decode_attention(_p(q), _p(k_cache), _p(v_cache), dtype, batch, q_heads, kv_heads,
                                head_dim, capacity, valid, _p(out))
    return out


def paged_attention(q, k_pool, v_pool, dtype: int, q_heads: int, kv_heads: int, head_dim: int,
                    page_size: int, page_stride: int, head_stride: int, block_tables,
                    max_pages: int, valid_lengths, active_count: int):
    q, k_pool, v_pool = _c(q, dtype), _c(k_pool, dtype), _c(v_pool, dtype)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    vl = np.ascontiguousarray(valid_lengths, dtype=np.int32)
    batch = vl.size
    out = np.zeros((batch, q_heads * head_dim), dtype=np.float64)
    written = np.zeros((batch, q_heads), dtype=np.uint8)
    lib().tmco_paged_attention(_p(q), _p(k_pool), _p(v_pool), dtype, batch, q_heads, kv_heads,
                               head_dim, page_size, page_stride, head_stride, _p(bt), max_pages,
                               _p(vl), active_count, _p(out), _p(written))
    return out, written.astype(bool)


def causal_prefill_attention(q, k_pool, v_pool, dtype: int, q_heads: int, kv_heads: int,
                             head_dim: int, page_size: int, page_stride: int, head_stride: int,
                             block_table, max_pages: int, valid: int, chunk: int,
                             active_count: int | None = None):
    """Causal chunk attention of emitPagedKVAttention with causalPrefill
    (KVCacheMetalEmitter.cpp:159-163, queryLength = chunk): query row r of a
    chunk of ``chunk`` tokens attends ``valid - chunk + r + 1`` positions of
    one request's pages, ``valid`` being the cache length with the chunk
    appended.  Each row is tmco_paged_attention at that length over the
    request's one block table; returns (out [chunk, q_heads*D], written)."""
    lengths = np.array([valid - chunk + r + 1 for r in range(chunk)], np.int32)
    tables = np.tile(np.asarray(block_table, np.int32).reshape(1, max_pages), (chunk, 1))
    return paged_attention(q, k_pool, v_pool, dtype, q_heads, kv_heads, head_dim, page_size,
                           page_stride, head_stride, tables, max_pages, lengths,
                           chunk if active_count is None else active_count)


def argmax(logits) -> np.ndarray:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rows, vocab = x.shape
    out = np.empty(rows, dtype=np.int32)
    lib().tmco_argmax(_p(x), rows, vocab, _p(out))
    return out


def append_contiguous(inp, cache, batch, heads, head_dim, seq_len, capacity, head_major, valid):
    inp = np.ascontiguousarray(inp, dtype=np.uint16)
    out = np.array(cache, dtype=np.uint16, copy=True)
    lib().tmco_append_contiguous(_p(inp), batch, heads, head_dim, seq_len, capacity,
                                 int(head_major), valid, _p(out))
    return out


def append_paged(inp, cache, batch, heads, head_dim, seq_len, capacity, page_size, head_major,
                 valid, block_table):
    inp = np.ascontiguousarray(inp, dtype=np.uint16)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    out = np.array(cache, dtype=np.uint16, copy=True)
    lib().tmco_append_paged(_p(inp), batch, heads, head_dim, seq_len, capacity, page_size,
                            int(head_major), valid, _p(bt), _p(out))
    return out


def append_serving(inp, cache, max_batch, heads, head_dim, capacity, page_size, head_major,
                   valid_lengths, block_tables, active_count):
    inp = np.ascontiguousarray(inp, dtype=np.uint16)
    vl = np.ascontiguousarray(valid_lengths, dtype=np.int32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    out = np.array(cache, dtype=np.uint16, copy=True)
    lib().tmco_append_serving(_p(inp), max_batch, heads, head_dim, capacity, page_size,
                              int(head_major), _p(vl), _p(bt), active_count, _p(out))
    return out


# ---------------------------------------------------------------- decode step
class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in
                ("input_norm", "wq", "wk", "wv", "wo", "post_norm", "wg", "wu", "wd")]


class _Model(C.Structure):
    _fields_ = [("layers", C.c_size_t), ("hidden", C.c_size_t), ("heads", C.c_size_t),
                ("head_dim", C.c_size_t), ("intermediate", C.c_size_t),
                ("vocabulary", C.c_size_t), ("capacity", C.c_size_t), ("epsilon", C.c_float),
                ("kv_heads", C.c_size_t), ("embedding", C.c_void_p), ("final_norm", C.c_void_p), ("lm_head", C.c_void_p),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
                ("layer", C.POINTER(_Layer))]


def linear_values(x_bits, weight) -> np.ndarray:
    """tmco_linear_values: the same double sums as linear(x, w, F16) for fp16
    bits x and W, computed by the decode step's blocked, threaded linear."""
    x = decode(np.ascontiguousarray(x_bits, dtype=np.uint16), F16)
    w = np.ascontiguousarray(weight, dtype=np.uint16)
    rows, k = x.reshape(-1, w.shape[1]).shape
    y = np.empty((rows, w.shape[0]), dtype=np.float64)
    lib().tmco_linear_values(_p(x), _p(w), rows, k, w.shape[0], _p(y))
    return y


def set_threads(threads: int) -> None:
    """Threads of decoder_step (default 1); results do not depend on it."""
    lib().tmco_set_threads(int(threads))


def decoder_step(weights: dict, cfg: dict, key_pools, value_pools, page_size: int,
                 max_pages: int, block_tables, tokens, valid_lengths, layer_limit: int = 0,
                 logits_from: int = 0):
    """One decode step (tmco_decoder_step).  ``weights`` holds fp16 bit arrays:
    embedding, final_norm, lm_head, rope_cos/rope_sin (fp32) and ``layers`` (a
    list of dicts with input_norm, wq, wk, wv, wo, post_norm, wg, wu, wd).
    Pools are lists (one per layer) of uint16 arrays updated in place."""
    keep = []
    layers = (_Layer * cfg["layers"])()
    for i, lw in enumerate(weights["layers"]):
        for name in _Layer._fields_:
            arr = np.ascontiguousarray(lw[name[0]], dtype=np.uint16)
            keep.append(arr)
            setattr(layers[i], name[0], arr.ctypes.data)
    top = {}
    for name in ("embedding", "final_norm", "lm_head"):
        top[name] = np.ascontiguousarray(weights[name], dtype=np.uint16)
    for name in ("rope_cos", "rope_sin"):
        top[name] = np.ascontiguousarray(weights[name], dtype=np.float32)
    m = _Model(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["head_dim"], cfg["intermediate"],
               cfg["vocabulary"], cfg["capacity"], cfg["epsilon"], cfg.get("kv_heads", 0),
               top["embedding"].ctypes.data,
               top["final_norm"].ctypes.data, top["lm_head"].ctypes.data,
               top["rope_cos"].ctypes.data, top["rope_sin"].ctypes.data, layers)
    for p in list(key_pools) + list(value_pools):
        assert p.dtype == np.uint16 and p.flags.c_contiguous
    kp = (C.c_void_p * len(key_pools))(*[p.ctypes.data for p in key_pools])
    vp = (C.c_void_p * len(value_pools))(*[p.ctypes.data for p in value_pools])
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    tk = np.ascontiguousarray(tokens, dtype=np.int32)
    vl = np.ascontiguousarray(valid_lengths, dtype=np.int32)
    batch = tk.size
    logits = np.zeros((batch, cfg["vocabulary"]), dtype=np.float32)
    nxt = np.zeros(batch, dtype=np.int32)
    rc = lib().tmco_decoder_step(C.byref(m), kp, vp, page_size, max_pages, _p(bt), _p(tk), _p(vl),
                                 batch, layer_limit, logits_from, _p(logits), _p(nxt))
    if rc != 0:
        raise ValueError(f"tmco_decoder_step failed with {rc}")
    return logits, nxt
