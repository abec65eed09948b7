"""CPU checks of the boundary: the built library loads and exports every
function include/tmc_hip.h declares; argument validation fails loudly
before touching a device."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header="tmc_hip.h"):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(tmc_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


HEADERS = sorted(h for h in os.listdir(os.path.join(ROOT, "include")) if h.endswith(".h"))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("tmc_gemv_f16", "tmc_skinny_gemm_f16_mfma", "tmc_rmsnorm", "tmc_add_rmsnorm",
                     "tmc_silu_mul", "tmc_gate_up_silu_f16", "tmc_kv_append", "tmc_paged_kv_append",
                     "tmc_decode_attention", "tmc_paged_decode_attention", "tmc_rt_create",
                     "tmc_buf_create", "tmc_kernel_resolve", "tmc_prepare", "tmc_exec_run",
                     "tmc_seq_create", "tmc_seq_run", "tmc_last_error"):
        assert required in names


@pytest.mark.parametrize("header", HEADERS)
def test_library_exports_every_declared_symbol(tmc, header):
    lib = tmc.lib()
    missing = [n for n in declared_functions(header) if not hasattr(lib, n)]
    assert not missing, f"{header}: missing exports: {missing}"


def test_bench_helpers_stay_out_of_the_boundary():
    """The measurement helpers (synthetic fill, copy and gather probes, the
    attention timeline) are declared in tmc_bench.h, not in the drop-in
    header."""
    boundary, bench = set(declared_functions()), set(declared_functions("tmc_bench.h"))
    assert bench == {"tmc_fill_normal", "tmc_copy_bytes", "tmc_read_probe",
                     "tmc_paged_gather_probe", "tmc_attention_timeline"}
    assert not boundary & bench


def test_argument_validation_fails_before_device_work(tmc):
    lib = tmc.lib()
    assert lib.tmc_gemv_f16(None, None, None, 1, 1, 8, 8, None) != 0
    assert "null" in tmc.last_error()
    assert lib.tmc_rmsnorm(C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), 1, 1, 8, -1.0, None) != 0
    assert "epsilon" in tmc.last_error()
    assert lib.tmc_decode_attention(C.c_void_p(16), C.c_void_p(16), C.c_void_p(16),
                                    C.c_void_p(16), C.c_void_p(16), 0, 1, 32, 8, 96, 64, None, 0,
                                    None) != 0
    assert "head_dim" in tmc.last_error()
    with pytest.raises(tmc.TmcError):
        tmc.check(lib.tmc_silu_mul(None, None, None, 0, 4, None), "silu")
    # the decode-step fusions and the staged / device copies
    p = C.c_void_p(16)
    assert lib.tmc_qkv_rope_append_f16(None, p, p, p, p, p, p, p, p, p, 64, 2, 1, 16, 32, 16, None,
                                       None) != 0
    assert "null" in tmc.last_error()
    assert lib.tmc_qkv_rope_append_f16(p, p, p, p, p, p, p, p, p, p, 64, 3, 2, 16, 32, 16, None,
                                       None) != 0
    assert "head geometry" in tmc.last_error()
    bad_cfg = tmc.GemvConfig(1, 1, 4, 4)  # the RoPE epilogue needs two rows per wave
    assert lib.tmc_qkv_rope_append_f16(p, p, p, p, p, p, p, p, p, p, 64, 2, 1, 16, 32, 16,
                                       C.byref(bad_cfg), None) != 0
    assert "rows_per_wave 2" in tmc.last_error()
    assert lib.tmc_qkv_rope_append_packed_f16(p, p, p, p, p, p, p, p, p, p, 4, 64, 2, 1, 16, 32, 16,
                                              2, tmc.Y_PACKED, None, None) != 0
    assert "layout" in tmc.last_error()
    # a block-table row shorter than ceil(capacity / page_size) would let a
    # request index the next request's row
    assert lib.tmc_qkv_rope_append_packed_f16(p, p, p, p, p, p, p, p, p, p, 4, 64, 2, 1, 16, 32, 16,
                                              1, 0, None, None) != 0
    assert "ceil(capacity / page_size)" in tmc.last_error()
    assert lib.tmc_add_rmsnorm_qkv_rope_append_f16(p, p, p, p, None, p, p, p, p, p, p, p, p, 64, 2,
                                                   1, 16, 32, 16, 1e-6, None, None) != 0
    assert "null" in tmc.last_error()
    assert lib.tmc_buf_write_raw_async(None, p, 1, 0) != 0
    assert "invalid range" in tmc.last_error()
    assert lib.tmc_buf_write_sparse_async(None, p, 1) != 0
    assert "null buffer" in tmc.last_error()
    # graph-path element-wise kernels: the tuner's workgroup sizes only
    assert lib.tmc_elementwise(0, p, p, p, 0, 64, 512, None) != 0
    assert "threads must be 64, 128 or 256" in tmc.last_error()
    assert lib.tmc_elementwise(1, p, None, p, 0, 64, 64, None) != 0
    assert "null" in tmc.last_error()
    # the gather probe takes the attention's geometry rules
    assert lib.tmc_paged_gather_probe(p, p, p, p, 16, 8, 64, 16, 256, 8192, 16384, 2048, p,
                                      None) != 0
    assert "head_dim must be 128" in tmc.last_error()
    assert lib.tmc_paged_gather_probe(p, p, p, None, 16, 8, 128, 16, 256, 8192, 16384, 2048, p,
                                      None) != 0
    assert "null" in tmc.last_error()
    # the attention timeline exists only in the TMC_ATTN_TIMELINE build
    assert lib.tmc_attention_timeline(p, 16) != 0
    assert "TMC_ATTN_TIMELINE" in tmc.last_error()
    # the residual epilogue: batch 1 only, fp16 operands present
    assert lib.tmc_gemv_residual_f16(p, p, None, p, 1, 64, 8, None, None) != 0
    assert "null" in tmc.last_error()
    assert lib.tmc_gemv_residual_f16(p, p, p, p, 2, 64, 8, None, None) != 0
    assert "batch must be 1" in tmc.last_error()
    # the fused norm holds at most 8192 features (four 16-byte chunks a lane)
    assert lib.tmc_add_rmsnorm_gemv_f16(p, None, p, p, None, p, 0, 1, 8200, 8, C.c_float(1e-6),
                                        None, None) != 0
    assert "up to 8192" in tmc.last_error()
    cfg = tmc.GemvConfig(1, 1, 2, 2)  # the norm fusion maps waves to norm groups at k split 4
    assert lib.tmc_add_rmsnorm_gemv_f16(p, None, p, p, None, p, 0, 1, 4096, 8, C.c_float(1e-6),
                                        C.byref(cfg), None) != 0
    assert "k_split 4" in tmc.last_error()
    assert lib.tmc_buf_copy_async(None, 0, None, 0, 1) != 0
    assert "different runtimes" in tmc.last_error()


def test_packed_folded_norm_and_residual_validation(tmc):
    """The folded-norm packed entry points need epsilon > 0 and at most 4
    waves per tile; the residual epilogue writes fp16 and needs a residual."""
    lib = tmc.lib()
    p = C.c_void_p(256)
    assert lib.tmc_gemm_packed_norm_f16(p, p, p, 0, 16, 4096, 4096, C.c_float(0.0), 1, None,
                                        None) != 0
    assert "epsilon" in tmc.last_error()
    cfg = tmc.GemvConfig(3, 1, 2, 8)
    assert lib.tmc_gate_up_silu_packed_norm_f16(p, p, p, p, 16, 4096, 11008, C.c_float(1e-6), 3,
                                                C.byref(cfg), None) != 0
    assert "1..4 with RMSNorm" in tmc.last_error()
    assert lib.tmc_rmsnorm_qkv_rope_append_packed_f16(p, p, p, p, p, p, p, p, p, p, 16, 512, 8, 4,
                                                      64, 64, 16, 4, C.c_float(-1.0), 1, None,
                                                      None) != 0
    assert "epsilon" in tmc.last_error()
    assert lib.tmc_gemm_packed_residual_f16(p, p, None, p, 16, 4096, 4096, 2, None, None) != 0
    assert "residual" in tmc.last_error()
    assert lib.tmc_pack_weights_scaled_f16(None, p, p, 8, 8, None) != 0
    assert "null" in tmc.last_error()


def test_attention_output_fusion_limits(tmc):
    """tmc_paged_attention_output_f16 refuses what its one-launch form cannot
    hold, before any device work: (q, k, v, lengths, tables, active, W,
    residual, y, q_heads, kv_heads, head_dim, page, max_pages, pool_pages,
    page_stride, head_stride, out, workspace, bytes, stream)."""
    lib = tmc.lib()
    p = C.c_void_p(256)
    ws = tmc.attention_output_workspace_bytes(32, 32, 4096)
    # arrival counters (8 slices of 512 rows, padded to 256 bytes) + the
    # kv heads' fp32 partial sums [32][4096]
    assert ws == 256 + 32 * 4096 * 4
    assert tmc.attention_output_workspace_bytes(8, 4, 512) == 256 + 4 * 512 * 4
    assert tmc.attention_output_workspace_bytes(32, 8, 4096) == 0  # group 4
    assert tmc.attention_output_workspace_bytes(4, 4, 100) == 0  # no slice height divides 100

    def call(q_heads=32, kv_heads=32, head_dim=128, page=16, max_pages=64, pool_pages=96,
             out=4096, workspace=p, nbytes=ws, weight=p):
        page_stride = kv_heads * page * head_dim
        return lib.tmc_paged_attention_output_f16(
            p, p, p, p, p, None, weight, None, p, q_heads, kv_heads, head_dim, page, max_pages,
            pool_pages, page_stride, page * head_dim, out, workspace, nbytes, None)

    assert call(weight=None) != 0 and "null" in tmc.last_error()
    assert call(head_dim=64) != 0 and "head_dim must be 128" in tmc.last_error()
    assert call(kv_heads=8) != 0 and "1 or 2" in tmc.last_error()
    assert call(page=8, max_pages=128) != 0 and "multiple of 16" in tmc.last_error()
    assert call(max_pages=65) != 0 and "at most 1024" in tmc.last_error()
    assert call(pool_pages=0) != 0 and "known number of pages" in tmc.last_error()
    assert call(out=100) != 0 and "multiple of 128" in tmc.last_error()
    assert call(nbytes=ws - 4) != 0 and "workspace" in tmc.last_error()
    assert call(workspace=None) != 0 and "workspace" in tmc.last_error()


def test_paged_attention_output_layout_validation(tmc):
    """tmc_paged_decode_attention_ex accepts layout 0 or TMC_LAYOUT_Y_PACKED
    (fp16 only) and refuses anything else before any device work."""
    lib = tmc.lib()
    p = C.c_void_p(256)
    ws = tmc.attention_workspace_bytes(4, 8, 8, 128, 4096)

    def call(layout, dtype=0):
        return lib.tmc_paged_decode_attention_ex(p, p, p, p, p, None, p, dtype, 4, 8, 8, 128, 16,
                                                 256, 512, 8 * 16 * 128, 16 * 128, p, ws, layout,
                                                 None)

    assert call(3) != 0 and "layout must be 0 or TMC_LAYOUT_Y_PACKED" in tmc.last_error()
    assert call(tmc.X_PACKED) != 0 and "layout" in tmc.last_error()
    assert call(tmc.Y_PACKED, dtype=1) != 0 and "fp16" in tmc.last_error()


def test_attention_workspace_sizes(tmc):
    # Every workspace starts with a fixed 64 KiB area of arrival counters
    # (one int32 per (request, kv head)), the same for every head size, then
    # the [request][q head][split][D + 2] fp32 partials.
    area = 64 << 10
    # VALU kernel (D=64): one split of 256 positions needs no workspace
    assert tmc.attention_workspace_bytes(2, 8, 8, 64, 256) == 0
    assert tmc.attention_workspace_bytes(2, 8, 8, 64, 1024) == area + 2 * 8 * 4 * 66 * 4
    # D = 128: chunk = pow2 in [128, 1024] not above batch * kv_heads * capacity / 256
    assert tmc.attention_workspace_bytes(16, 32, 8, 128, 4096) == area + 16 * 32 * 4 * 130 * 4
    assert tmc.attention_workspace_bytes(1, 32, 32, 128, 4096) == area + 1 * 32 * 8 * 130 * 4
    # capacity <= 1024 with a GQA group <= 2: one 16-wave block per row, no
    # workspace; a group of 4 keeps the split layout
    assert tmc.attention_workspace_bytes(1, 32, 32, 128, 1024) == 0
    assert tmc.attention_workspace_bytes(1, 8, 4, 128, 1024) == 0
    assert tmc.attention_workspace_bytes(1, 8, 2, 128, 1024) == area + 1 * 8 * 8 * 130 * 4
    assert tmc.attention_workspace_bytes(1, 8, 8, 128, 128) == 0
    # more than 16384 (request, kv head) rows: the counter area grows to one
    # int32 per row, rounded up to 256 bytes
    assert tmc.attention_workspace_bytes(4100, 8, 8, 64, 1024) == \
        (4100 * 8 * 4 + 255) // 256 * 256 + 4100 * 8 * 4 * 66 * 4
    # bad head ratio
    assert tmc.attention_workspace_bytes(2, 6, 4, 64, 1024) == 0
