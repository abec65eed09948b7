"""The product's host conversions (tmc_host_encode / tmc_host_decode in
libtmc_hip.so, the code behind tmc_buf_create / tmc_buf_write /
tmc_buf_read) against the reference's storeValue golden vectors
(GraphReference.cpp:39-87, MetalRuntime.mm:42-104), exhaustively over every
fp16 bit pattern, and against the oracle's separate bit-field restatement on
random and boundary floats.  CPU only: these functions touch no device."""
import numpy as np
import pytest

F16, F32, BF16, I32 = 0, 1, 2, 3


def _same_values(got, exp):
    got, exp = np.asarray(got, np.float32), np.asarray(exp, np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(exp))
    m = ~np.isnan(exp)
    assert np.array_equal(got[m].view(np.uint32), exp[m].view(np.uint32))


def test_fp16_upload_matches_reference_golden_ties(tmc, golden):
    x = golden["store_in"]
    bits = tmc.host_encode(x, F16)
    _same_values(tmc.host_decode(bits, F16), golden["store_f16"])
    nan = np.isnan(x)
    assert np.array_equal(bits[nan] & 0x7fff, np.full(nan.sum(), 0x7e00, np.uint16))


def test_fp16_decode_every_bit_pattern(tmc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = tmc.host_decode(bits, F16)
    _same_values(got, bits.view(np.float16).astype(np.float32))
    signs = (got.view(np.uint32) >> 31).astype(np.uint16)
    assert np.array_equal(signs, bits >> 15)  # signed zeros and NaNs keep their sign
    finite = ~np.isnan(got)
    assert np.array_equal(tmc.host_encode(got[finite], F16), bits[finite])


def test_fp16_encode_matches_oracle_restatement(tmc, orc):
    rng = np.random.default_rng(11)
    scales = [1e-8, 6e-8, 3e-5, 6.1e-5, 1.0, 2.0 ** 10, 6e4, 65504.0, 65519.0, 65520.0, 1e6]
    parts = [rng.standard_normal(200000).astype(np.float32) * np.float32(s) for s in scales]
    # exact fp16 ties, in the normal and the subnormal range
    h = rng.integers(0, 0x7bff, 50000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    parts.append(((lo.astype(np.float64) + hi) / 2).astype(np.float32))
    parts.append(np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -np.nan, 2.0 ** -25, -2.0 ** -25,
                           2.0 ** -26, 65520.0, -65520.0, 65519.996, 1e-45, -1e-45], np.float32))
    x = np.concatenate(parts)
    ours = tmc.host_encode(x, F16)
    theirs = orc.f16(x)
    assert np.array_equal(ours, theirs)


def test_bf16_and_int32_uploads(tmc, orc, golden):
    import torch
    rng = np.random.default_rng(12)
    x = rng.standard_normal(100000).astype(np.float32) * np.float32(100)
    x[::7] = np.round(x[::7])  # exact integers and values with a zero low half
    bits = tmc.host_encode(x, BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, ref)
    assert np.array_equal(bits, orc.encode(x, BF16))
    _same_values(tmc.host_decode(bits, BF16), orc.decode(bits, BF16))
    ints = tmc.host_encode(golden["store_i32_in"], I32)
    assert np.array_equal(ints.astype(np.float32), golden["store_i32"])
    assert np.array_equal(tmc.host_decode(ints, I32), golden["store_i32"])


def test_host_conversion_errors(tmc):
    import ctypes as C
    lib = tmc.lib()
    assert lib.tmc_host_encode(None, 4, F16, None) != 0
    assert "null" in tmc.last_error()
    assert lib.tmc_host_decode(C.c_void_p(16), 1, 9, C.c_void_p(16)) != 0
    assert "dtype" in tmc.last_error()
    assert lib.tmc_host_encode(None, 0, F16, None) == 0


@pytest.mark.gpu
def test_buffer_upload_bits_match_reference_ties(tmc, orc, golden):
    """tmc_buf_create and tmc_buf_write (with an offset) store the golden
    fp16 bits; tmc_buf_read returns the reference's stored values."""
    import ctypes as C
    rt = tmc.Runtime()
    x = golden["store_in"]
    buf = rt.create_buffer(x.size, F16, x)
    raw = np.empty(x.size, np.uint16)
    tmc.check(tmc.lib().tmc_buf_read_raw(buf.handle, raw.ctypes.data_as(C.c_void_p), x.size, 0),
              "tmc_buf_read_raw")
    assert np.array_equal(raw, orc.f16(x))
    _same_values(buf.read(), golden["store_f16"])
    big = rt.create_buffer(x.size + 5, F16)
    assert np.isnan(big.read()).all()  # fresh float buffers hold the NaN sentinel
    big.write(x, 5)
    back = big.read()
    assert np.isnan(back[:5]).all()
    _same_values(back[5:], golden["store_f16"])
    ib = rt.create_buffer(golden["store_i32_in"].size, I32, golden["store_i32_in"])
    assert np.array_equal(ib.read(), golden["store_i32"])
