"""Python front end of the gfx950 decode backend (libtmc_hip.so).

The product is the C ABI declared in include/tmc_hip.h; this module binds it
with ctypes so tests, bench.py and __graft_entry__ can drive it with torch
device tensors.  torch is imported before the library is opened so that the
library binds to the HIP runtime torch already loaded (one runtime per
process).  There is no fallback: if the library is missing or fails to load,
every call raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtmc_hip.so")

F16, F32, BF16, I32 = 0, 1, 2, 3

_lib = None


class TmcError(RuntimeError):
    pass


def build() -> str:
    from importlib import util
    spec = util.spec_from_file_location("tmc_build", os.path.join(HERE, "build.py"))
    mod = util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build()


def _declare(l):
    vp, i64, sz, i32, f, d = C.c_void_p, C.c_int64, C.c_size_t, C.c_int, C.c_float, C.c_double
    sigs = {
        "tmc_last_error": (C.c_char_p, []),
        "tmc_gemv_f16": (i32, [vp, vp, vp, i32, i64, i64, i64, vp]),
        "tmc_skinny_gemm_f16_mfma": (i32, [vp, vp, vp, i32, i64, i64, i64, vp]),
        "tmc_gemv_f16_config": (i32, [vp, vp, vp, i32, i64, i64, i64, vp, vp]),
        "tmc_qkv_rope_append_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64,
                                          i64, i64, i64, vp, vp]),
        "tmc_qkv_rope_append_packed_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64,
                                                 i64, i64, i64, i64, i64, i64, i32, vp, vp]),
        "tmc_add_rmsnorm_qkv_rope_append_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                                      vp, vp, i64, i64, i64, i64, i64, i64,
                                                      C.c_float, vp, vp]),
        "tmc_gate_up_silu_f16_config": (i32, [vp, vp, vp, vp, i64, i64, i64, vp, vp]),
        "tmc_gemv_default_config": (i32, [i64, i64, i64, i32, vp]),
        "tmc_gate_up_silu_f16": (i32, [vp, vp, vp, vp, i64, i64, i64, vp]),
        "tmc_rmsnorm": (i32, [vp, vp, vp, i32, i64, i64, f, vp]),
        "tmc_add_rmsnorm": (i32, [vp, vp, vp, vp, vp, i32, i64, i64, f, vp]),
        "tmc_add_rmsnorm_gemv_f16": (i32, [vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, f, vp, vp]),
        "tmc_gemv_residual_f16": (i32, [vp, vp, vp, vp, i64, i64, i64, vp, vp]),
        "tmc_add_rmsnorm_gate_up_silu_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, f, vp,
                                                   vp]),
        "tmc_add_rmsnorm_ex": (i32, [vp, vp, vp, vp, vp, i32, i64, i64, f, i32, vp]),
        "tmc_packed_activation_elements": (C.c_int64, [i64, i64]),
        "tmc_pack_activations_f16": (i32, [vp, vp, i64, i64, i32, vp]),
        "tmc_gemm_packed_ex_f16": (i32, [vp, vp, vp, i32, i64, i64, i64, i32, vp, vp]),
        "tmc_gate_up_silu_packed_ex_f16": (i32, [vp, vp, vp, vp, i64, i64, i64, i32, vp, vp]),
        "tmc_packed_weight_elements": (C.c_int64, [i64, i64]),
        "tmc_pack_weights_f16": (i32, [vp, vp, i64, i64, vp]),
        "tmc_gemm_packed_f16": (i32, [vp, vp, vp, i32, i64, i64, i64, vp, vp]),
        "tmc_gate_up_silu_packed_f16": (i32, [vp, vp, vp, vp, i64, i64, i64, vp, vp]),
        "tmc_rmsnorm_threads": (i32, [vp, vp, vp, i32, i64, i64, f, i32, i32, vp]),
        "tmc_add_rmsnorm_threads": (i32, [vp, vp, vp, vp, vp, i32, i64, i64, f, i32, i32, vp]),
        "tmc_silu_mul": (i32, [vp, vp, vp, i32, i64, vp]),
        "tmc_add": (i32, [vp, vp, vp, i32, i64, vp]),
        "tmc_embedding": (i32, [vp, vp, vp, i32, i64, i64, i64, vp]),
        "tmc_rope": (i32, [vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, vp]),
        "tmc_serving_rope": (i32, [vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, vp]),
        "tmc_kv_append": (i32, [vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, vp]),
        "tmc_paged_kv_append": (i32, [vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, i32, vp]),
        "tmc_serving_kv_append": (i32, [vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, vp]),
        "tmc_decode_rope_append": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64,
                                         i64, i64, i64, i64, vp]),
        "tmc_prefill_rope_append": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64,
                                          i64, i64, i64, i64, vp]),
        "tmc_prefill_rope_append_rows": (i32, [vp, vp, vp, vp, vp, vp, i64, vp, vp, vp, vp, i32,
                                               i64, i64, i64, i64, i64, i64, i64, vp]),
        "tmc_prefill_attention_rows_f16": (i32, [vp, vp, vp, vp, vp, vp, i64, vp, vp, i64, i64,
                                                 i64, i64, i64, i64, i64, i64, i64, vp]),
        "tmc_gemm_rows_workspace_bytes": (sz, []),
        "tmc_gemm_rows_f16": (i32, [vp, vp, vp, i32, i64, i64, i64, vp, sz, vp]),
        "tmc_gemm_mfma_f16": (i32, [vp, vp, vp, i32, i64, i64, i64, vp]),
        "tmc_prefill_attention_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64,
                                            i64, i64, i64, i64, vp]),
        "tmc_attention_workspace_bytes": (sz, [i64, i64, i64, i64, i64]),
        "tmc_decode_attention": (i32, [vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, vp, sz,
                                       vp]),
        "tmc_paged_decode_attention": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64,
                                             i64, i64, i64, i64, i64, vp, sz, vp]),
        "tmc_paged_decode_attention_ex": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64,
                                                i64, i64, i64, i64, i64, i64, vp, sz, i32, vp]),
        "tmc_paged_decode_attention_noalloc": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i64, i64,
                                                     i64, i64, i64, i64, i64, i64, i64, vp]),
        "tmc_attention_scratch_bytes": (sz, []),
        "tmc_gemm_packed_norm_f16": (i32, [vp, vp, vp, i32, i64, i64, i64, f, i32, vp, vp]),
        "tmc_gate_up_silu_packed_norm_f16": (i32, [vp, vp, vp, vp, i64, i64, i64, f, i32, vp,
                                                   vp]),
        "tmc_rmsnorm_qkv_rope_append_packed_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                                         i64, i64, i64, i64, i64, i64, i64, i64,
                                                         f, i32, vp, vp]),
        "tmc_pack_weights_scaled_f16": (i32, [vp, vp, vp, i64, i64, vp]),
        "tmc_gemm_packed_residual_f16": (i32, [vp, vp, vp, vp, i64, i64, i64, i32, vp, vp]),
        "tmc_attention_output_workspace_bytes": (sz, [i64, i64, i64]),
        "tmc_paged_attention_output_f16": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64,
                                                 i64, i64, i64, i64, i64, i64, i64, vp, sz, vp]),
        "tmc_paged_gather_probe": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, i64, i64,
                                         vp, vp]),
        "tmc_attention_timeline": (i32, [vp, i64]),
        "tmc_argmax_f32": (i32, [vp, vp, i64, i64, vp]),
        "tmc_lm_head_argmax_workspace_bytes": (sz, [i64, i64]),
        "tmc_rmsnorm_lm_head_partial_argmax_f16": (i32, [vp, vp, vp, vp, sz, i64, i64, f, vp, vp]),
        "tmc_lm_head_partial_argmax_packed_norm_f16": (i32, [vp, vp, vp, sz, i64, i64, i64, f, i32,
                                                              vp, vp]),
        "tmc_lm_head_final_argmax": (i32, [vp, sz, vp, i64, i64, vp]),
        "tmc_fill_normal": (i32, [vp, i32, i64, C.c_uint64, f, f, vp]),
        "tmc_copy_bytes": (i32, [vp, vp, sz, vp]),
        "tmc_read_probe": (i32, [vp, sz, vp, vp]),
        "tmc_elementwise": (i32, [i32, vp, vp, vp, i32, i64, i32, vp]),
        "tmc_rt_create": (i32, [C.POINTER(vp)]),
        "tmc_rt_destroy": (None, [vp]),
        "tmc_rt_is_available": (i32, [vp]),
        "tmc_rt_device_name": (C.c_char_p, [vp]),
        "tmc_rt_init_error": (C.c_char_p, [vp]),
        "tmc_rt_stream": (vp, [vp]),
        "tmc_rt_fail_next": (None, [vp, i32]),
        "tmc_buf_create": (i32, [vp, sz, i32, vp, C.POINTER(vp)]),
        "tmc_buf_wrap": (i32, [vp, vp, sz, i32, C.POINTER(vp)]),
        "tmc_buf_write": (i32, [vp, vp, sz, sz]),
        "tmc_buf_write_raw": (i32, [vp, vp, sz, sz]),
        "tmc_buf_write_raw_async": (i32, [vp, vp, sz, sz]),
        "tmc_buf_write_sparse_async": (i32, [vp, vp, sz]),
        "tmc_decode_chain": (i32, [vp, vp, vp, vp, i64, vp]),
        "tmc_buf_copy_async": (i32, [vp, sz, vp, sz, sz]),
        "tmc_buf_read_raw": (i32, [vp, vp, sz, sz]),
        "tmc_buf_read": (i32, [vp, vp]),
        "tmc_buf_count": (sz, [vp]),
        "tmc_buf_dtype": (i32, [vp]),
        "tmc_buf_device_ptr": (vp, [vp]),
        "tmc_buf_release": (None, [vp]),
        "tmc_host_encode": (i32, [vp, sz, i32, vp]),
        "tmc_host_decode": (i32, [vp, sz, i32, vp]),
        "tmc_kernel_resolve": (i32, [vp, C.c_char_p, C.POINTER(vp), C.POINTER(i32), vp, vp]),
        "tmc_kernel_dispatch": (i32, [vp, C.POINTER(sz), C.POINTER(sz)]),
        "tmc_kernel_release": (None, [vp]),
        "tmc_prepare": (i32, [vp, vp, vp, sz, vp, sz, sz, sz, vp, sz, C.POINTER(vp)]),
        "tmc_exec_run": (i32, [vp, i32, C.POINTER(d), C.POINTER(d)]),
        "tmc_exec_release": (None, [vp]),
        "tmc_seq_create": (i32, [vp, vp, sz, C.POINTER(vp)]),
        "tmc_seq_run": (i32, [vp, C.POINTER(d), C.POINTER(d)]),
        "tmc_seq_launch": (i32, [vp]),
        "tmc_seq_release": (None, [vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def lib() -> C.CDLL:
    """Open libtmc_hip.so (raises TmcError when it is missing)."""
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401  (binds one HIP runtime per process)
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise TmcError(f"{LIB_PATH} is missing; run aicompiler-test_amd/build.py")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def open_variant(name: str) -> C.CDLL:
    """Another build of the same ABI next to libtmc_hip.so (for example
    libtmc_hip_merge_launch.so), declared like the main library.  Tests swap
    it in for lib() to run the same checks against that build."""
    lib()  # the main library first: one HIP runtime, bound through torch
    path = os.path.join(os.path.dirname(LIB_PATH), name)
    if not os.path.exists(path):
        raise TmcError(f"{path} is missing; run aicompiler-test_amd/build.py")
    variant = C.CDLL(path)
    _declare(variant)
    return variant


_host = None


def host():
    """The C++ host layer as a Python module (_tmc_host, built next to this
    file).  torch is imported first so one HIP runtime serves the process."""
    global _host
    if _host is None:
        import importlib.util
        import sysconfig
        lib()  # loads torch's HIP runtime and libtmc_hip.so first
        path = os.path.join(HERE, "_tmc_host" + sysconfig.get_config_var("EXT_SUFFIX"))
        if not os.path.exists(path):
            raise TmcError(f"{path} is missing; run aicompiler-test_amd/build.py")
        spec = importlib.util.spec_from_file_location("_tmc_host", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _host = mod
    return _host


def last_error() -> str:
    return lib().tmc_last_error().decode()


def check(rc: int, what: str = "tmc call") -> None:
    if rc != 0:
        raise TmcError(f"{what}: {last_error()}")


# ---------------------------------------------------------------- torch helpers
def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _dtype_code(t) -> int:
    import torch
    return {torch.float16: F16, torch.float32: F32, torch.bfloat16: BF16,
            torch.int32: I32}[t.dtype]


def gemv(x, w, y, stream=None):
    """y = x @ w.T (fp16 x, w; y fp16 or fp32)."""
    b, k = x.shape
    n = w.shape[0]
    check(lib().tmc_gemv_f16(_ptr(x), _ptr(w), _ptr(y), _dtype_code(y), b, k, n, _stream(stream)),
          "tmc_gemv_f16")


class GemvConfig(C.Structure):
    """tmc_gemv_config (include/tmc_hip.h)."""
    _fields_ = [("algorithm", C.c_int), ("rows_per_wave", C.c_int), ("unroll", C.c_int),
                ("k_split", C.c_int)]

    def astuple(self):
        return (self.algorithm, self.rows_per_wave, self.unroll, self.k_split)


def default_config(batch, in_features, out_features, gated=False) -> GemvConfig:
    cfg = GemvConfig()
    check(lib().tmc_gemv_default_config(batch, in_features, out_features, int(gated),
                                        C.byref(cfg)), "tmc_gemv_default_config")
    return cfg


def gemv_config(x, w, y, cfg, stream=None):
    b, k = x.shape
    n = w.shape[0]
    check(lib().tmc_gemv_f16_config(_ptr(x), _ptr(w), _ptr(y), _dtype_code(y), b, k, n,
                                    C.byref(cfg), _stream(stream)), "tmc_gemv_f16_config")


def gate_up_silu_config(x, wg, wu, out, cfg, stream=None):
    b, h = x.shape
    f = wg.shape[0]
    check(lib().tmc_gate_up_silu_f16_config(_ptr(x), _ptr(wg), _ptr(wu), _ptr(out), b, h, f,
                                            C.byref(cfg), _stream(stream)),
          "tmc_gate_up_silu_f16_config")


def add_rmsnorm_gemv(residual, update, gamma, w, sum_out, y, eps, cfg=None, stream=None):
    """Batch-1 GEMV of RMSNorm(residual + update) (update None: RMSNorm(residual))."""
    b, k = residual.shape
    n = w.shape[0]
    check(lib().tmc_add_rmsnorm_gemv_f16(_ptr(residual), _ptr(update) if update is not None else None,
                                         _ptr(gamma), _ptr(w),
                                         _ptr(sum_out) if sum_out is not None else None, _ptr(y),
                                         _dtype_code(y), b, k, n, eps,
                                         C.byref(cfg) if cfg is not None else None,
                                         _stream(stream)), "tmc_add_rmsnorm_gemv_f16")


def gemv_residual(x, w, residual, y, cfg=None, stream=None):
    """Batch-1 y = h(h(W x) + residual) (the o / down projections of the
    folded decode step)."""
    b, k = x.shape
    n = w.shape[0]
    check(lib().tmc_gemv_residual_f16(_ptr(x), _ptr(w), _ptr(residual), _ptr(y), b, k, n,
                                      C.byref(cfg) if cfg is not None else None, _stream(stream)),
          "tmc_gemv_residual_f16")


def add_rmsnorm_gate_up_silu(residual, update, gamma, wg, wu, sum_out, out, eps, cfg=None,
                             stream=None):
    b, h = residual.shape
    f = wg.shape[0]
    check(lib().tmc_add_rmsnorm_gate_up_silu_f16(
        _ptr(residual), _ptr(update) if update is not None else None, _ptr(gamma), _ptr(wg),
        _ptr(wu), _ptr(sum_out) if sum_out is not None else None, _ptr(out), b, h, f, eps,
        C.byref(cfg) if cfg is not None else None, _stream(stream)),
        "tmc_add_rmsnorm_gate_up_silu_f16")


X_PACKED, Y_PACKED = 1, 2  # TMC_LAYOUT_X_PACKED, TMC_LAYOUT_Y_PACKED


def packed_activation_elements(rows, cols) -> int:
    return int(lib().tmc_packed_activation_elements(rows, cols))


def pack_activations(x, out=None, unpack=False, rows=None, cols=None, stream=None):
    """Row-major fp16 [rows, cols] <-> fragment order (tmc_pack_activations_f16)."""
    import torch
    if unpack:
        assert out is not None and rows is not None and cols is not None
    else:
        rows, cols = x.shape
        if out is None:
            out = torch.empty(packed_activation_elements(rows, cols), dtype=torch.float16,
                              device=x.device)
    check(lib().tmc_pack_activations_f16(_ptr(x), _ptr(out), rows, cols, int(unpack),
                                         _stream(stream)), "tmc_pack_activations_f16")
    return out


def add_rmsnorm_ex(residual, update, w, sum_out, norm_out, eps, layout, rows=None, width=None,
                   stream=None):
    rows = rows if rows is not None else residual.shape[0]
    width = width if width is not None else residual.shape[1]
    check(lib().tmc_add_rmsnorm_ex(_ptr(residual), _ptr(update) if update is not None else None,
                                   _ptr(w), _ptr(sum_out) if sum_out is not None else None,
                                   _ptr(norm_out), _dtype_code(residual), rows, width, eps, layout,
                                   _stream(stream)), "tmc_add_rmsnorm_ex")


def gemm_packed_ex(x, packed, y, batch, in_features, out_features, layout, cfg=None, y_dtype=None,
                   stream=None):
    check(lib().tmc_gemm_packed_ex_f16(_ptr(x), _ptr(packed), _ptr(y),
                                       _dtype_code(y) if y_dtype is None else y_dtype, batch,
                                       in_features, out_features, layout,
                                       C.byref(cfg) if cfg is not None else None, _stream(stream)),
          "tmc_gemm_packed_ex_f16")


def gate_up_silu_packed_ex(x, packed_gate, packed_up, out, batch, hidden, intermediate, layout,
                           cfg=None, stream=None):
    check(lib().tmc_gate_up_silu_packed_ex_f16(_ptr(x), _ptr(packed_gate), _ptr(packed_up),
                                               _ptr(out), batch, hidden, intermediate, layout,
                                               C.byref(cfg) if cfg is not None else None,
                                               _stream(stream)), "tmc_gate_up_silu_packed_ex_f16")


def _cfg_ref(cfg):
    if cfg is None:
        return None
    return C.byref(GemvConfig(*cfg) if isinstance(cfg, tuple) else cfg)


def gemm_packed_norm(x, packed_scaled, y, batch, in_features, out_features, eps, layout,
                     cfg=None, stream=None):
    """Packed GEMM of RMSNorm(x) * gamma with the norm folded in; the weights
    come from pack_weights(w, gamma=...) (tmc_gemm_packed_norm_f16)."""
    check(lib().tmc_gemm_packed_norm_f16(_ptr(x), _ptr(packed_scaled), _ptr(y), _dtype_code(y),
                                         batch, in_features, out_features, eps, layout,
                                         _cfg_ref(cfg), _stream(stream)),
          "tmc_gemm_packed_norm_f16")


def gate_up_silu_packed_norm(x, packed_gate, packed_up, out, batch, hidden, intermediate, eps,
                             layout, cfg=None, stream=None):
    check(lib().tmc_gate_up_silu_packed_norm_f16(_ptr(x), _ptr(packed_gate), _ptr(packed_up),
                                                 _ptr(out), batch, hidden, intermediate, eps,
                                                 layout, _cfg_ref(cfg), _stream(stream)),
          "tmc_gate_up_silu_packed_norm_f16")


def rmsnorm_qkv_rope_append_packed(x, packed_scaled, cos, sin, valid_lengths, tables, active,
                                   q_out, k_pool, v_pool, batch, hidden, q_heads, kv_heads,
                                   head_dim, capacity, page_size, max_pages, eps, layout=0,
                                   config=None, stream=None):
    check(lib().tmc_rmsnorm_qkv_rope_append_packed_f16(
        _ptr(x), _ptr(packed_scaled), _ptr(cos), _ptr(sin), _ptr(valid_lengths), _ptr(tables),
        _ptr(active), _ptr(q_out), _ptr(k_pool), _ptr(v_pool), batch, hidden, q_heads, kv_heads,
        head_dim, capacity, page_size, max_pages, eps, layout, _cfg_ref(config),
        _stream(stream)), "tmc_rmsnorm_qkv_rope_append_packed_f16")


def gemm_packed_residual(x, packed, residual, y, batch, in_features, out_features, layout,
                         cfg=None, stream=None):
    """y = fp16(fp16(x W^T) + residual) over packed W (tmc_gemm_packed_residual_f16)."""
    check(lib().tmc_gemm_packed_residual_f16(_ptr(x), _ptr(packed), _ptr(residual), _ptr(y),
                                             batch, in_features, out_features, layout,
                                             _cfg_ref(cfg), _stream(stream)),
          "tmc_gemm_packed_residual_f16")


def packed_weight_elements(out_features, in_features) -> int:
    return int(lib().tmc_packed_weight_elements(out_features, in_features))


def pack_weights(w, packed=None, stream=None, gamma=None):
    """Fragment-packed copy of fp16 W [out, in] (tmc_pack_weights_f16); with
    gamma, of W . diag(gamma) (tmc_pack_weights_scaled_f16)."""
    import torch
    n, k = w.shape
    if packed is None:
        packed = torch.empty(packed_weight_elements(n, k), dtype=torch.float16, device=w.device)
    check(lib().tmc_pack_weights_scaled_f16(_ptr(w), _ptr(gamma), _ptr(packed), n, k,
                                            _stream(stream)), "tmc_pack_weights_scaled_f16")
    return packed


def gemm_packed(x, packed, y, out_features, cfg=None, stream=None):
    b, k = x.shape
    check(lib().tmc_gemm_packed_f16(_ptr(x), _ptr(packed), _ptr(y), _dtype_code(y), b, k,
                                    out_features, C.byref(cfg) if cfg is not None else None,
                                    _stream(stream)), "tmc_gemm_packed_f16")


def gate_up_silu_packed(x, packed_gate, packed_up, out, intermediate, cfg=None, stream=None):
    b, h = x.shape
    check(lib().tmc_gate_up_silu_packed_f16(_ptr(x), _ptr(packed_gate), _ptr(packed_up), _ptr(out),
                                            b, h, intermediate,
                                            C.byref(cfg) if cfg is not None else None,
                                            _stream(stream)), "tmc_gate_up_silu_packed_f16")


def skinny_gemm(x, w, y, stream=None):
    b, k = x.shape
    n = w.shape[0]
    check(lib().tmc_skinny_gemm_f16_mfma(_ptr(x), _ptr(w), _ptr(y), _dtype_code(y), b, k, n,
                                         _stream(stream)), "tmc_skinny_gemm_f16_mfma")


def gate_up_silu(x, wg, wu, out, stream=None):
    b, h = x.shape
    f = wg.shape[0]
    check(lib().tmc_gate_up_silu_f16(_ptr(x), _ptr(wg), _ptr(wu), _ptr(out), b, h, f,
                                     _stream(stream)), "tmc_gate_up_silu_f16")


def rmsnorm(x, w, y, eps, stream=None):
    rows, width = x.shape
    check(lib().tmc_rmsnorm(_ptr(x), _ptr(w), _ptr(y), _dtype_code(x), rows, width, eps,
                            _stream(stream)), "tmc_rmsnorm")


def add_rmsnorm(residual, update, w, sum_out, norm_out, eps, stream=None):
    rows, width = residual.shape
    check(lib().tmc_add_rmsnorm(_ptr(residual), _ptr(update), _ptr(w), _ptr(sum_out),
                                _ptr(norm_out), _dtype_code(residual), rows, width, eps,
                                _stream(stream)), "tmc_add_rmsnorm")


def rmsnorm_threads(x, w, y, eps, threads, variant=0, stream=None):
    """tmc_rmsnorm_threads: threads 64..1024, variant 0 default / 1 two-pass."""
    rows, width = x.shape
    check(lib().tmc_rmsnorm_threads(_ptr(x), _ptr(w), _ptr(y), _dtype_code(x), rows, width, eps,
                                    threads, variant, _stream(stream)), "tmc_rmsnorm_threads")


def add_rmsnorm_threads(residual, update, w, sum_out, norm_out, eps, threads, variant=0,
                        stream=None):
    rows, width = residual.shape
    check(lib().tmc_add_rmsnorm_threads(_ptr(residual), _ptr(update), _ptr(w), _ptr(sum_out),
                                        _ptr(norm_out), _dtype_code(residual), rows, width, eps,
                                        threads, variant, _stream(stream)),
          "tmc_add_rmsnorm_threads")


def silu_mul(gate, up, out, stream=None):
    check(lib().tmc_silu_mul(_ptr(gate), _ptr(up), _ptr(out), _dtype_code(gate), gate.numel(),
                             _stream(stream)), "tmc_silu_mul")


def add(a, b, out, stream=None):
    check(lib().tmc_add(_ptr(a), _ptr(b), _ptr(out), _dtype_code(a), a.numel(), _stream(stream)),
          "tmc_add")


def embedding(tokens, table, out, stream=None):
    vocab, hidden = table.shape
    check(lib().tmc_embedding(_ptr(tokens), _ptr(table), _ptr(out), _dtype_code(table),
                              tokens.numel(), hidden, vocab, _stream(stream)), "tmc_embedding")


def rope(x, cos, sin, valid_length, out, batch, seq, heads, head_dim, capacity, stream=None):
    check(lib().tmc_rope(_ptr(x), _ptr(cos), _ptr(sin), _ptr(valid_length), _ptr(out),
                         _dtype_code(x), batch, seq, heads, head_dim, capacity, _stream(stream)),
          "tmc_rope")


def serving_rope(x, cos, sin, valid_lengths, active, out, max_batch, heads, head_dim, capacity,
                 stream=None):
    check(lib().tmc_serving_rope(_ptr(x), _ptr(cos), _ptr(sin), _ptr(valid_lengths), _ptr(active),
                                 _ptr(out), _dtype_code(x), max_batch, heads, head_dim, capacity,
                                 _stream(stream)), "tmc_serving_rope")


def kv_append(inp, valid_length, cache, batch, seq, heads, head_dim, capacity, head_major,
              stream=None):
    check(lib().tmc_kv_append(_ptr(inp), _ptr(valid_length), _ptr(cache), _dtype_code(inp), batch,
                              seq, heads, head_dim, capacity, int(head_major), _stream(stream)),
          "tmc_kv_append")


def paged_kv_append(inp, valid_length, table, cache, batch, seq, heads, head_dim, capacity,
                    page_size, head_major, stream=None):
    check(lib().tmc_paged_kv_append(_ptr(inp), _ptr(valid_length), _ptr(table), _ptr(cache),
                                    _dtype_code(inp), batch, seq, heads, head_dim, capacity,
                                    page_size, int(head_major), _stream(stream)),
          "tmc_paged_kv_append")


def serving_kv_append(inp, valid_lengths, tables, active, cache, max_batch, heads, head_dim,
                      capacity, page_size, head_major, stream=None):
    check(lib().tmc_serving_kv_append(_ptr(inp), _ptr(valid_lengths), _ptr(tables), _ptr(active),
                                      _ptr(cache), _dtype_code(inp), max_batch, heads, head_dim,
                                      capacity, page_size, int(head_major), _stream(stream)),
          "tmc_serving_kv_append")


def decode_rope_append(qkv, cos, sin, valid_lengths, tables, active, q_out, k_pool, v_pool,
                       max_batch, q_heads, kv_heads, head_dim, capacity, page_size, max_pages,
                       stream=None):
    check(lib().tmc_decode_rope_append(_ptr(qkv), _ptr(cos), _ptr(sin), _ptr(valid_lengths),
                                       _ptr(tables), _ptr(active), _ptr(q_out), _ptr(k_pool),
                                       _ptr(v_pool), _dtype_code(qkv), max_batch, q_heads,
                                       kv_heads, head_dim, capacity, page_size, max_pages,
                                       _stream(stream)),
          "tmc_decode_rope_append")


def qkv_rope_append(x, w, cos, sin, valid_lengths, table, active, q_out, k_pool, v_pool, q_heads,
                    kv_heads, head_dim, capacity, page_size, config=None, stream=None):
    """Batch-1 q.k.v projection x @ w.T with RoPE and the paged K/V append
    fused in its epilogue (tmc_qkv_rope_append_f16)."""
    cfg = None
    if config is not None:
        cfg = GemvConfig(*config) if isinstance(config, tuple) else config
    check(lib().tmc_qkv_rope_append_f16(_ptr(x), _ptr(w), _ptr(cos), _ptr(sin), _ptr(valid_lengths),
                                        _ptr(table), _ptr(active), _ptr(q_out), _ptr(k_pool),
                                        _ptr(v_pool), x.shape[-1], q_heads, kv_heads, head_dim,
                                        capacity, page_size, None if cfg is None else C.byref(cfg),
                                        _stream(stream)),
          "tmc_qkv_rope_append_f16")


def qkv_rope_append_packed(x, packed_w, cos, sin, valid_lengths, tables, active, q_out, k_pool,
                           v_pool, batch, hidden, q_heads, kv_heads, head_dim, capacity, page_size,
                           max_pages, layout=0, config=None, stream=None):
    """Batched q.k.v projection over packed weights with RoPE and the paged
    append in its epilogue (tmc_qkv_rope_append_packed_f16)."""
    cfg = None
    if config is not None:
        cfg = GemvConfig(*config) if isinstance(config, tuple) else config
    check(lib().tmc_qkv_rope_append_packed_f16(
        _ptr(x), _ptr(packed_w), _ptr(cos), _ptr(sin), _ptr(valid_lengths), _ptr(tables),
        _ptr(active), _ptr(q_out), _ptr(k_pool), _ptr(v_pool), batch, hidden, q_heads, kv_heads,
        head_dim, capacity, page_size, max_pages, layout, None if cfg is None else C.byref(cfg),
        _stream(stream)), "tmc_qkv_rope_append_packed_f16")


def add_rmsnorm_qkv_rope_append(residual, update, gamma, w, sum_out, cos, sin, valid_lengths,
                                table, active, q_out, k_pool, v_pool, q_heads, kv_heads, head_dim,
                                capacity, page_size, eps, config=None, stream=None):
    """qkv_rope_append of RMSNorm(residual + update) * gamma (update None:
    RMSNorm(residual) * gamma), the norm built inside the kernel."""
    cfg = None
    if config is not None:
        cfg = GemvConfig(*config) if isinstance(config, tuple) else config
    check(lib().tmc_add_rmsnorm_qkv_rope_append_f16(
        _ptr(residual), _ptr(update) if update is not None else None, _ptr(gamma), _ptr(w),
        _ptr(sum_out) if sum_out is not None else None, _ptr(cos), _ptr(sin), _ptr(valid_lengths),
        _ptr(table), _ptr(active), _ptr(q_out), _ptr(k_pool), _ptr(v_pool), residual.shape[-1],
        q_heads, kv_heads, head_dim, capacity, page_size, eps,
        None if cfg is None else C.byref(cfg), _stream(stream)),
        "tmc_add_rmsnorm_qkv_rope_append_f16")


def prefill_rope_append(qkv, cos, sin, valid_lengths, table, active, q_out, k_pool, v_pool, rows,
                        q_heads, kv_heads, head_dim, capacity, page_size, max_pages, stream=None):
    check(lib().tmc_prefill_rope_append(_ptr(qkv), _ptr(cos), _ptr(sin), _ptr(valid_lengths),
                                        _ptr(table), _ptr(active), _ptr(q_out), _ptr(k_pool),
                                        _ptr(v_pool), _dtype_code(qkv), rows, q_heads, kv_heads,
                                        head_dim, capacity, page_size, max_pages, _stream(stream)),
          "tmc_prefill_rope_append")


def prefill_rope_append_rows(qkv, cos, sin, valid_lengths, tables, row_table, active, q_out,
                             k_pool, v_pool, rows, q_heads, kv_heads, head_dim, capacity,
                             page_size, max_pages, stream=None):
    """tables [table_rows, max_pages]; row_table [rows] int32."""
    check(lib().tmc_prefill_rope_append_rows(
        _ptr(qkv), _ptr(cos), _ptr(sin), _ptr(valid_lengths), _ptr(tables), _ptr(row_table),
        tables.shape[0], _ptr(active), _ptr(q_out), _ptr(k_pool), _ptr(v_pool), _dtype_code(qkv),
        rows, q_heads, kv_heads, head_dim, capacity, page_size, max_pages, _stream(stream)),
        "tmc_prefill_rope_append_rows")


def prefill_attention_rows(q, k_pool, v_pool, valid_lengths, tables, row_table, active, out, rows,
                           q_heads, kv_heads, head_dim, page_size, max_pages, page_stride,
                           head_stride, stream=None, pool_pages=None):
    if pool_pages is None:
        pool_pages = min(k_pool.numel(), v_pool.numel()) // page_stride
    check(lib().tmc_prefill_attention_rows_f16(
        _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(valid_lengths), _ptr(tables), _ptr(row_table),
        tables.shape[0], _ptr(active), _ptr(out), rows, q_heads, kv_heads, head_dim, page_size,
        max_pages, pool_pages, page_stride, head_stride, _stream(stream)),
        "tmc_prefill_attention_rows_f16")


def gemm_rows_workspace_bytes() -> int:
    return int(lib().tmc_gemm_rows_workspace_bytes())


def gemm_rows(x, w, y, workspace=None, stream=None):
    """y[m, n] = x[m, k] w[n, k]^T on the MFMA GEMM (fp16 in, fp32 accumulation;
    K split over the workspace when the tiles alone leave CUs idle)."""
    m, k = x.shape
    n = w.shape[0]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().tmc_gemm_rows_f16(_ptr(x), _ptr(w), _ptr(y), _dtype_code(y), m, k, n,
                                  _ptr(workspace), ws_bytes, _stream(stream)), "tmc_gemm_rows_f16")


def gemm_mfma(x, w, y, stream=None):
    """y[m, n] = x[m, k] w[n, k]^T on the hand-written gfx950 MFMA GEMM."""
    m, k = x.shape
    n = w.shape[0]
    check(lib().tmc_gemm_mfma_f16(_ptr(x), _ptr(w), _ptr(y), _dtype_code(y), m, k, n,
                                  _stream(stream)), "tmc_gemm_mfma_f16")


def prefill_attention(q, k_pool, v_pool, valid_lengths, table, active, out, rows, q_heads,
                      kv_heads, head_dim, page_size, max_pages, page_stride, head_stride,
                      stream=None, pool_pages=None):
    """Causal chunk attention over one request's pages; pool_pages defaults
    to the pages the k_pool tensor holds."""
    if pool_pages is None:
        pool_pages = min(k_pool.numel(), v_pool.numel()) // page_stride
    check(lib().tmc_prefill_attention_f16(
        _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(valid_lengths), _ptr(table), _ptr(active),
        _ptr(out), rows, q_heads, kv_heads, head_dim, page_size, max_pages, pool_pages,
        page_stride, head_stride, _stream(stream)), "tmc_prefill_attention_f16")


def attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, capacity) -> int:
    return int(lib().tmc_attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, capacity))


def decode_attention(q, k_cache, v_cache, valid_length, out, batch, q_heads, kv_heads, head_dim,
                     capacity, workspace=None, stream=None):
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().tmc_decode_attention(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(valid_length),
                                     _ptr(out), _dtype_code(q), batch, q_heads, kv_heads, head_dim,
                                     capacity, _ptr(workspace), ws_bytes, _stream(stream)),
          "tmc_decode_attention")


def paged_gather_probe(k_pool, v_pool, valid_lengths, tables, batch, kv_heads, head_dim,
                       page_size, max_pages, page_stride, head_stride, sink, stream=None):
    """Load-only pass over the K/V bytes paged attention reads (bandwidth probe)."""
    pool_pages = min(k_pool.numel(), v_pool.numel()) // page_stride
    check(lib().tmc_paged_gather_probe(
        _ptr(k_pool), _ptr(v_pool), _ptr(valid_lengths), _ptr(tables), batch, kv_heads, head_dim,
        page_size, max_pages, pool_pages, page_stride, head_stride, _ptr(sink), _stream(stream)),
        "tmc_paged_gather_probe")


def paged_decode_attention(q, k_pool, v_pool, valid_lengths, tables, active, out, max_batch,
                           q_heads, kv_heads, head_dim, page_size, max_pages, page_stride,
                           head_stride, workspace=None, stream=None, pool_pages=None,
                           layout=0):
    """pool_pages defaults to the pages the k_pool tensor holds; layout
    Y_PACKED writes out in the packed activation order."""
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if pool_pages is None:
        pool_pages = min(k_pool.numel(), v_pool.numel()) // page_stride
    check(lib().tmc_paged_decode_attention_ex(
        _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(valid_lengths), _ptr(tables), _ptr(active),
        _ptr(out), _dtype_code(q), max_batch, q_heads, kv_heads, head_dim, page_size, max_pages,
        pool_pages, page_stride, head_stride, _ptr(workspace), ws_bytes, layout,
        _stream(stream)),
        "tmc_paged_decode_attention")


def attention_output_workspace_bytes(q_heads, kv_heads, out_features):
    return lib().tmc_attention_output_workspace_bytes(q_heads, kv_heads, out_features)


def paged_attention_output(q, k_pool, v_pool, valid_lengths, tables, active, weight, residual,
                           y, q_heads, kv_heads, head_dim, page_size, max_pages, page_stride,
                           head_stride, workspace, stream=None, pool_pages=None):
    """Batch-1 paged attention + output projection (+ residual unless None).
    `workspace` must be zero before its first use (the kernel leaves its
    arrival counters at zero after every call)."""
    if pool_pages is None:
        pool_pages = min(k_pool.numel(), v_pool.numel()) // page_stride
    ws_bytes = workspace.numel() * workspace.element_size()
    check(lib().tmc_paged_attention_output_f16(
        _ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(valid_lengths), _ptr(tables), _ptr(active),
        _ptr(weight), _ptr(residual), _ptr(y), q_heads, kv_heads, head_dim, page_size, max_pages,
        pool_pages, page_stride, head_stride, weight.shape[0], _ptr(workspace), ws_bytes,
        _stream(stream)), "tmc_paged_attention_output_f16")


def argmax(logits, tokens, stream=None):
    rows, vocab = logits.shape
    check(lib().tmc_argmax_f32(_ptr(logits), _ptr(tokens), rows, vocab, _stream(stream)),
          "tmc_argmax_f32")


def lm_head_argmax_workspace_bytes(rows, vocabulary) -> int:
    return int(lib().tmc_lm_head_argmax_workspace_bytes(rows, vocabulary))


def rmsnorm_lm_head_argmax(residual, gamma, w, workspace, tokens, eps, cfg=None, stream=None):
    """Token-only batch-1 LM head: partial argmax of W * RMSNorm(residual)
    (tmc_rmsnorm_lm_head_partial_argmax_f16), then the final argmax."""
    _, k = residual.shape
    n = w.shape[0]
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().tmc_rmsnorm_lm_head_partial_argmax_f16(
        _ptr(residual), _ptr(gamma), _ptr(w), _ptr(workspace), nbytes, k, n, eps, _cfg_ref(cfg),
        _stream(stream)), "tmc_rmsnorm_lm_head_partial_argmax_f16")
    check(lib().tmc_lm_head_final_argmax(_ptr(workspace), nbytes, _ptr(tokens), 1, n,
                                         _stream(stream)), "tmc_lm_head_final_argmax")


def lm_head_argmax_packed_norm(x, packed_scaled, workspace, tokens, batch, in_features,
                               vocabulary, eps, layout=0, cfg=None, stream=None):
    """Token-only batch > 1 LM head on packed gamma-scaled weights: partial
    argmax (tmc_lm_head_partial_argmax_packed_norm_f16), then the final."""
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().tmc_lm_head_partial_argmax_packed_norm_f16(
        _ptr(x), _ptr(packed_scaled), _ptr(workspace), nbytes, batch, in_features, vocabulary, eps,
        layout, _cfg_ref(cfg), _stream(stream)), "tmc_lm_head_partial_argmax_packed_norm_f16")
    check(lib().tmc_lm_head_final_argmax(_ptr(workspace), nbytes, _ptr(tokens), batch,
                                         vocabulary, _stream(stream)), "tmc_lm_head_final_argmax")


def fill_normal(t, seed, mean=0.0, std=1.0, stream=None):
    check(lib().tmc_fill_normal(_ptr(t), _dtype_code(t), t.numel(), seed, mean, std,
                                _stream(stream)), "tmc_fill_normal")


def read_probe(src, nbytes, sink, stream=None):
    """tmc_read_probe (include/tmc_bench.h): read nbytes of src once."""
    check(lib().tmc_read_probe(_ptr(src), nbytes, _ptr(sink), _stream(stream)), "tmc_read_probe")


def copy_bytes(src, dst, nbytes, stream=None):
    check(lib().tmc_copy_bytes(_ptr(src), _ptr(dst), nbytes, _stream(stream)), "tmc_copy_bytes")


# ---------------------------------------------------------------- host conversions
def host_encode(values, dtype: int):
    """fp32 -> storage bits with the runtime's upload rule (tmc_host_encode)."""
    import numpy as np
    src = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(src.shape, dtype={F16: np.uint16, BF16: np.uint16, F32: np.float32,
                                     I32: np.int32}[dtype])
    check(lib().tmc_host_encode(src.ctypes.data_as(C.c_void_p), src.size, dtype,
                                out.ctypes.data_as(C.c_void_p)), "tmc_host_encode")
    return out


def host_decode(bits, dtype: int):
    """Storage bits -> fp32 with the runtime's readback rule (tmc_host_decode)."""
    import numpy as np
    src = np.ascontiguousarray(bits, dtype={F16: np.uint16, BF16: np.uint16, F32: np.float32,
                                            I32: np.int32}[dtype])
    out = np.empty(src.shape, dtype=np.float32)
    check(lib().tmc_host_decode(src.ctypes.data_as(C.c_void_p), src.size, dtype,
                                out.ctypes.data_as(C.c_void_p)), "tmc_host_decode")
    return out


# ---------------------------------------------------------------- runtime objects
class Runtime:
    """Python mirror of tensor::metal::MetalRuntime over the tmc_rt_* ABI
    (MetalRuntime.hpp:149-208): buffers, kernel resolution, prepared
    executions and HIP-graph sequences on the runtime's own stream."""

    def __init__(self):
        self._h = C.c_void_p()
        check(lib().tmc_rt_create(C.byref(self._h)), "tmc_rt_create")

    def close(self):
        if self._h:
            lib().tmc_rt_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def is_available(self) -> bool:
        return bool(lib().tmc_rt_is_available(self._h))

    def device_name(self) -> str:
        return lib().tmc_rt_device_name(self._h).decode()

    def initialization_error(self) -> str:
        return lib().tmc_rt_init_error(self._h).decode()

    def stream_handle(self) -> int:
        return lib().tmc_rt_stream(self._h) or 0

    def torch_stream(self):
        import torch
        return torch.cuda.ExternalStream(self.stream_handle())

    def fail_next(self, count: int) -> None:
        lib().tmc_rt_fail_next(self._h, count)

    def create_buffer(self, count: int, dtype: int, data=None) -> "Buffer":
        import numpy as np
        h = C.c_void_p()
        src = None
        if data is not None:
            src = np.ascontiguousarray(data, dtype=np.float32)
            assert src.size == count
        check(lib().tmc_buf_create(self._h, count, dtype,
                                   None if src is None else src.ctypes.data_as(C.c_void_p),
                                   C.byref(h)), "tmc_buf_create")
        return Buffer(h, self)

    def wrap(self, tensor) -> "Buffer":
        h = C.c_void_p()
        check(lib().tmc_buf_wrap(self._h, C.c_void_p(tensor.data_ptr()), tensor.numel(),
                                 _dtype_code(tensor), C.byref(h)), "tmc_buf_wrap")
        b = Buffer(h, self)
        b._keep = tensor
        return b

    def resolve(self, key: str) -> "Kernel":
        h = C.c_void_p()
        n = C.c_int()
        types = (C.c_int * 32)()
        writable = (C.c_int * 32)()
        check(lib().tmc_kernel_resolve(self._h, key.encode(), C.byref(h), C.byref(n), types,
                                       writable), "tmc_kernel_resolve")
        return Kernel(h, [types[i] for i in range(n.value)],
                      [bool(writable[i]) for i in range(n.value)])

    def prepare(self, kernel: "Kernel", inputs, outputs, constants=()) -> "Exec":
        groups, threads = C.c_size_t(), C.c_size_t()
        check(lib().tmc_kernel_dispatch(kernel.handle, C.byref(groups), C.byref(threads)),
              "tmc_kernel_dispatch")
        ins = (C.c_void_p * max(len(inputs), 1))(*[b.handle for b in inputs])
        outs = (C.c_void_p * max(len(outputs), 1))(*[b.handle for b in outputs])
        consts = (C.c_uint32 * max(len(constants), 1))(*constants)
        h = C.c_void_p()
        check(lib().tmc_prepare(self._h, kernel.handle, ins, len(inputs), outs, len(outputs),
                                groups.value, threads.value, consts, len(constants),
                                C.byref(h)), "tmc_prepare")
        return Exec(h, list(inputs) + list(outputs))

    def sequence(self, steps) -> "Sequence":
        arr = (C.c_void_p * len(steps))(*[s.handle for s in steps])
        h = C.c_void_p()
        check(lib().tmc_seq_create(self._h, arr, len(steps), C.byref(h)), "tmc_seq_create")
        return Sequence(h, list(steps))


class Buffer:
    def __init__(self, handle, rt):
        self.handle, self.rt, self._keep = handle, rt, None

    def __del__(self):
        try:
            lib().tmc_buf_release(self.handle)
        except Exception:
            pass

    @property
    def count(self) -> int:
        return int(lib().tmc_buf_count(self.handle))

    @property
    def dtype(self) -> int:
        return int(lib().tmc_buf_dtype(self.handle))

    def write(self, data, offset: int = 0) -> None:
        import numpy as np
        src = np.ascontiguousarray(data, dtype=np.float32).ravel()
        check(lib().tmc_buf_write(self.handle, src.ctypes.data_as(C.c_void_p), src.size, offset),
              "tmc_buf_write")

    def read(self):
        import numpy as np
        out = np.empty(self.count, dtype=np.float32)
        check(lib().tmc_buf_read(self.handle, out.ctypes.data_as(C.c_void_p)), "tmc_buf_read")
        return out

    def write_raw_async(self, data, offset: int = 0) -> None:
        """Raw storage bits queued on the runtime stream (no host wait);
        `data` may be reused as soon as this returns."""
        import numpy as np
        dt = {F16: np.uint16, BF16: np.uint16, F32: np.float32, I32: np.int32}[self.dtype]
        src = np.ascontiguousarray(data, dtype=dt).ravel()
        check(lib().tmc_buf_write_raw_async(self.handle, src.ctypes.data_as(C.c_void_p), src.size,
                                            offset), "tmc_buf_write_raw_async")

    def write_sparse_async(self, indices, values) -> None:
        """int32 values stored at increasing element indices, queued on the
        runtime stream (applied by a kernel that reads the staged pairs)."""
        import numpy as np
        pairs = np.stack([np.asarray(indices, np.int32).ravel(),
                          np.asarray(values, np.int32).ravel()], axis=1)
        pairs = np.ascontiguousarray(pairs)
        check(lib().tmc_buf_write_sparse_async(self.handle, pairs.ctypes.data_as(C.c_void_p),
                                               pairs.shape[0]), "tmc_buf_write_sparse_async")

    def read_raw(self):
        import numpy as np
        dt = {F16: np.uint16, BF16: np.uint16, F32: np.float32, I32: np.int32}[self.dtype]
        out = np.empty(self.count, dtype=dt)
        check(lib().tmc_buf_read_raw(self.handle, out.ctypes.data_as(C.c_void_p), self.count, 0),
              "tmc_buf_read_raw")
        return out


class Kernel:
    def __init__(self, handle, types, writable):
        self.handle, self.types, self.writable = handle, types, writable

    def __del__(self):
        try:
            lib().tmc_kernel_release(self.handle)
        except Exception:
            pass


class Exec:
    def __init__(self, handle, keep):
        self.handle, self._keep = handle, keep

    def __del__(self):
        try:
            lib().tmc_exec_release(self.handle)
        except Exception:
            pass

    def run(self, reset_outputs: bool = True):
        gpu, cpu = C.c_double(), C.c_double()
        check(lib().tmc_exec_run(self.handle, int(reset_outputs), C.byref(gpu), C.byref(cpu)),
              "tmc_exec_run")
        return gpu.value, cpu.value


class Sequence:
    def __init__(self, handle, steps):
        self.handle, self._steps = handle, steps

    def __del__(self):
        try:
            lib().tmc_seq_release(self.handle)
        except Exception:
            pass

    def run(self):
        gpu, cpu = C.c_double(), C.c_double()
        check(lib().tmc_seq_run(self.handle, C.byref(gpu), C.byref(cpu)), "tmc_seq_run")
        return gpu.value, cpu.value

    def launch(self):
        check(lib().tmc_seq_launch(self.handle), "tmc_seq_launch")
