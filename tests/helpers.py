"""Shared helpers for the parity tests: seeded inputs, device transfer of
fp16 bit patterns, and the tolerance checks stated by the north star
(fp32 outputs within 1e-4 relative error; fp16-path outputs within 2e-2
absolute error and 3e-3 relative RMS error)."""
import numpy as np

F16, F32, BF16, I32 = 0, 1, 2, 3


def normal(seed, shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def uniform(seed, shape, lo, hi):
    return np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)


def dev_f16(bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16)).cuda()


def dev(arr, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(arr))
    return (t if dtype is None else t.to(dtype)).cuda()


def bits(t):
    return t.detach().cpu().contiguous().numpy().view(np.uint16)


def values(t):
    import torch
    return t.detach().float().cpu().numpy()


def assert_f16_path(actual, reference, what=""):
    a = np.asarray(actual, np.float64).ravel()
    r = np.asarray(reference, np.float64).ravel()
    assert a.shape == r.shape, what
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    err = np.abs(a - r)
    rel_rms = np.sqrt(np.mean(err ** 2)) / max(np.sqrt(np.mean(r ** 2)), 1e-30)
    assert err.max() <= 2e-2, f"{what}: max abs err {err.max():.3e} > 2e-2"
    assert rel_rms <= 3e-3, f"{what}: relative RMS err {rel_rms:.3e} > 3e-3"
    return err.max(), rel_rms


F32_ATOL = 1e-5  # the fp32 (absolute, relative) pair: (1e-5, 1e-4), GraphExecutor.cpp:31-34


def assert_f32_rel(actual, reference, rel=1e-4, what="", atol=F32_ATOL):
    """The reference's element rule for fp32 outputs, |a - r| <= atol + rel * |r|
    for every element (validation/Validator.cpp:26, with GraphExecutor.cpp's
    fp32 tolerance pair 1e-5 / 1e-4 and RMSNormTuner.cpp:19-20's).  Both
    sides fp32-accumulate the same fp16 products, so only the summation order
    differs: at K = 4096 that moves an output by about 1e-6, well inside the
    1e-5 floor."""
    a = np.asarray(actual, np.float64).ravel()
    r = np.asarray(reference, np.float64).ravel()
    assert a.shape == r.shape, what
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    err = np.abs(a - r)
    bound = atol + rel * np.abs(r)
    worst = float(np.max(err / bound)) if err.size else 0.0
    i = int(np.argmax(err / bound)) if err.size else 0
    assert np.all(err <= bound), (
        f"{what}: element {i} expected {r[i]:.8g} got {a[i]:.8g} "
        f"(|err| {err[i]:.3e} > {atol} + {rel} * |expected|)")
    return worst
