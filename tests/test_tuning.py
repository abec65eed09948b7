"""Host logic of the gfx950 tuners and admission (no GPU): candidate sets,
the hardware filter, the 1.05x two-round admission rule and the RMSNorm
double-precision reference (DecodeGEMVTuner.cpp:162-304,
RMSNormTuner.cpp:159-309, Validator.cpp:40-66)."""
import numpy as np
import pytest


def test_decode_gemv_candidates_cover_gfx950_configs(host):
    c1 = [c.astuple() for c in host.decode_gemv_candidates(1)]
    dots = [c for c in c1 if c[0] == 1]
    assert len(dots) == 12 and len(c1) == 14
    assert {c[1] for c in dots} == {1, 2} and {c[2] for c in dots} == {2, 4}
    assert {c[3] for c in dots} == {1, 2, 4}
    assert sorted(c for c in c1 if c[0] == 5) == [(5, 1, 1, 4), (5, 2, 1, 4)]
    c16 = [c.astuple() for c in host.decode_gemv_candidates(16)]
    assert (3, 1, 1, 8) in c16 and (3, 2, 1, 2) in c16 and (2, 1, 2, 16) in c16
    assert all(c[0] in (2, 3) for c in c16)
    c8 = [c.astuple() for c in host.decode_gemv_candidates(8)]
    assert (1, 1, 2, 4) in c8  # the dot algorithm still covers 8 rows


def test_decode_gemv_workgroups_are_wave_multiples(host):
    for batch in (1, 8, 16):
        for c in host.decode_gemv_candidates(batch):
            assert host.decode_gemv_threads(c) % 64 == 0


def test_decode_gemv_hardware_filter(host):
    cfg = host.DecodeGEMVConfig
    ok = lambda c, batch=16, k=4096, n=4096: host.decode_gemv_hardware_filter(
        c, batch, k, n, 1024, 160 * 1024, 1 << 40)
    assert ok(cfg(3, 1, 1, 8)) == ""
    # the persistent dot: batch 1 and K <= 16384 only
    assert ok(cfg(5, 2, 1, 4), batch=1, k=16384) == ""
    assert "persistent" in ok(cfg(5, 1, 1, 4), batch=2)
    assert "persistent" in ok(cfg(5, 1, 1, 4), batch=1, k=16392)
    assert ok(cfg(3, 4, 1, 16)) == ""                      # 64 KiB of partials: at the limit
    assert host.decode_gemv_lds_bytes(16, cfg(3, 4, 1, 16)) == 64 * 1024
    assert "LDS" in ok(cfg(3, 8, 1, 16))                   # 128 KiB at 1024 threads
    assert "64" in ok(cfg(2, 4, 1, 8))                     # 2048 threads
    assert "multiple of 8" in ok(cfg(1, 1, 2, 4), batch=1, k=4097)
    assert ok(cfg(4, 1, 1, 1), batch=1, k=4097) == ""     # the baseline takes any K
    assert "8 batch rows" in ok(cfg(1, 1, 2, 4), batch=16)
    assert "4 GiB" in ok(cfg(3, 1, 1, 4), batch=16, k=65536, n=65536)
    # a device with a smaller workgroup limit filters more
    assert host.decode_gemv_hardware_filter(cfg(3, 1, 1, 16), 16, 4096, 4096, 512, 65536,
                                            1 << 40) != ""


def test_decode_gemv_keys(host):
    cfg = host.DecodeGEMVConfig(3, 2, 1, 4)
    key = host.emit_decode_gemv_key(16, 4096, 12288, cfg, False)
    assert key == ("decode_gemv?batch=16&in=4096&out=12288&out_dtype=f16"
                   "&algorithm=3&rows_per_wave=2&unroll=1&k_split=4")
    assert host.emit_decode_gemv_key(1, 4096, 32000, host.DecodeGEMVConfig(), True) == \
        "decode_gemv?batch=1&in=4096&out=32000&out_dtype=f32"


@pytest.mark.parametrize("first,second,admitted,conservative", [
    ((True, 1.30), 1.10, True, 1.10),      # lower round ranks the candidate
    ((True, 1.06), 1.20, True, 1.06),
    ((True, 1.10), 1.04, False, 1.04),     # confirmation below 1.05x
    ((True, 1.049), None, False, 1.049),   # first round below: no confirmation taken
    ((True, 1.05), 1.05, True, 1.05),      # the bound itself admits
    ((False, 0.0), None, False, 0.0),
])
def test_admission_rule(host, first, second, admitted, conservative):
    ok, speed, reason = host.admission_decision(first[0], first[1], second)
    assert ok == admitted
    assert speed == pytest.approx(conservative)
    assert (reason == "") == admitted


def test_rms_norm_hardware_filter(host):
    assert host.rms_norm_hardware_filter(1, 4096, True, 64) == ""
    assert host.rms_norm_hardware_filter(1, 4096, False, 1024) == ""
    for bad in (0, 96, 2048):
        assert "64-lane" in host.rms_norm_hardware_filter(1, 4096, True, bad)


def test_rms_norm_reference_closed_form(host):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4097)).astype(np.float32)
    x[0] = 0.0
    x[1] *= 1e-4
    w = rng.uniform(0.5, 1.5, 4097).astype(np.float32)
    got = np.asarray(host.rms_norm_reference(3, 4097, 1e-6, x.ravel(), w)).reshape(3, 4097)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + np.float64(np.float32(1e-6))) * w
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15)
    assert np.all(got[0] == 0.0)
    # scale invariance up to the eps term: rmsnorm(c x) == rmsnorm(x) within
    # eps / (2 mean(x^2)) ~ 5e-7 relative for this row
    y = np.asarray(host.rms_norm_reference(1, 4097, 1e-6, (8.0 * x[2]).ravel(), w))
    np.testing.assert_allclose(y, got[2], rtol=1e-6)


def test_timing_statistics_and_paired_order(host):
    """benchmark::summarizeTimings / measurePair (Benchmark.cpp:51-95
    semantics): median and linearly interpolated 90th percentile of the
    samples, and paired rounds that alternate which arm runs first."""
    rng = np.random.default_rng(3)
    for n in (1, 2, 5, 31, 32):
        v = rng.uniform(1.0, 50.0, n)
        s = host.summarize_timings(list(v))
        assert s["samples"] == n and s["min_us"] == v.min() and s["max_us"] == v.max()
        assert abs(s["median_us"] - np.median(v)) <= 1e-12 * v.max()
        assert abs(s["p90_us"] - np.percentile(v, 90)) <= 1e-12 * v.max()
    assert host.summarize_timings([]) is None
    order = []
    times = {"b": iter([10.0, 12.0, 11.0, 13.0]), "c": iter([5.0, 6.0, 7.0, 8.0])}

    def arm(name):
        def run():
            order.append(name)
            return next(times[name])
        return run

    r = host.measure_pair(arm("b"), arm("c"), 4)
    assert r["passed"] and order == ["b", "c", "c", "b", "b", "c", "c", "b"]
    assert r["baseline"]["median_us"] == 11.5 and r["candidate"]["median_us"] == 6.5
    assert abs(r["speedup"] - 11.5 / 6.5) < 1e-12
    bad = host.measure_pair(lambda: 1.0, lambda: "device lost", 3)
    assert not bad["passed"] and bad["error"] == "Candidate: GPU execution failed: device lost"
    none = host.measure_pair(lambda: None, lambda: 1.0, 3)
    assert none["error"].startswith("Baseline: GPU timestamps unavailable")
    assert host.measure_pair(lambda: 1.0, lambda: 1.0, 0)["error"] == (
        "Benchmark requires at least one sample.")
