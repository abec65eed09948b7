"""tmc_paged_decode_attention_noalloc (static device scratch, no allocation)
against tmc_paged_decode_attention with a caller workspace, through the C
ABI: calls in a row, the second with a smaller input and two more of other
shapes whose split merge runs inside the partial kernel, each bit-identical
to the existing entry point on the same inputs (the two share their
kernels); limits beyond the scratch are rejected before any launch."""
import ctypes as C

import numpy as np
import pytest

from tests.helpers import dev, dev_f16, normal

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


def _case(orc, torch, seed, batch, qh, kvh, d, p, pages, max_pages, lo, hi):
    rng = np.random.default_rng(seed)
    k_pool = orc.f16(normal(seed + 1, (pages, kvh, p, d)))
    v_pool = orc.f16(normal(seed + 2, (pages, kvh, p, d)))
    q = orc.f16(normal(seed + 3, (batch, qh * d)))
    lengths = rng.integers(lo, hi + 1, batch).astype(np.int32)
    perm = rng.permutation(pages).astype(np.int32)
    tables = np.full((batch, max_pages), -1, np.int32)
    used = 0
    for r in range(batch):
        n = (int(lengths[r]) + p - 1) // p
        tables[r, :n] = perm[used:used + n]
        used += n
    return dict(q=dev_f16(q), k=dev_f16(k_pool), v=dev_f16(v_pool), lengths=dev(lengths),
                tables=dev(tables), active=torch.tensor([batch], dtype=torch.int32, device="cuda"),
                batch=batch, qh=qh, kvh=kvh, d=d, p=p, pages=pages, max_pages=max_pages)


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _run_both(tmc, torch, c):
    lib = tmc.lib()
    shape = (c["batch"], c["qh"] * c["d"])
    want = torch.full(shape, float("nan"), dtype=torch.float16, device="cuda")
    got = torch.full(shape, float("nan"), dtype=torch.float16, device="cuda")
    cap = c["p"] * c["max_pages"]
    need = tmc.attention_workspace_bytes(c["batch"], c["qh"], c["kvh"], c["d"], cap)
    ws = torch.zeros(max(need // 4, 1), dtype=torch.float32, device="cuda")
    page_stride, head_stride = c["kvh"] * c["p"] * c["d"], c["p"] * c["d"]
    tmc.check(lib.tmc_paged_decode_attention(
        _ptr(c["q"]), _ptr(c["k"]), _ptr(c["v"]), _ptr(c["lengths"]), _ptr(c["tables"]),
        _ptr(c["active"]), _ptr(want), 0, c["batch"], c["qh"], c["kvh"], c["d"], c["p"],
        c["max_pages"], c["pages"], page_stride, head_stride, _ptr(ws), need, None),
        "tmc_paged_decode_attention")
    tmc.check(lib.tmc_paged_decode_attention_noalloc(
        _ptr(c["q"]), _ptr(c["k"]), _ptr(c["v"]), _ptr(c["lengths"]), _ptr(c["tables"]),
        _ptr(c["active"]), _ptr(got), 0, c["batch"], c["qh"], c["kvh"], c["d"], c["p"],
        c["max_pages"], c["pages"], page_stride, head_stride, None),
        "tmc_paged_decode_attention_noalloc")
    torch.cuda.synchronize()
    return need, want, got


def test_noalloc_paged_attention_matches_workspace_entry(tmc, orc, torch):
    lib = tmc.lib()
    scratch = lib.tmc_attention_scratch_bytes()
    assert scratch == 16 << 20
    # C4's shape: 16 requests, GQA 32/8, D 128, 16-token pages, capacity 4096
    big = _case(orc, torch, 4100, 16, 32, 8, 128, 16, 4096, 256, 64, 4096)
    need, want, got = _run_both(tmc, torch, big)
    assert 0 < need <= scratch
    assert not torch.isnan(want).any()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # smaller second call: the scratch still holds the first call's partials
    small = _case(orc, torch, 4200, 5, 16, 4, 128, 16, 1024, 128, 1, 2048)
    need2, want2, got2 = _run_both(tmc, torch, small)
    assert 0 < need2 < need
    assert torch.equal(got2.view(torch.int16), want2.view(torch.int16))
    # GQA groups 4, 2 and 1 merge their splits inside the partial kernel
    # through arrival counters in a fixed area at the scratch's start (the
    # calls above are group 4): more shapes in a row (the scratch still holds
    # the earlier calls' slots), each finding the counters its predecessor
    # left at zero; group 8 merges in the combine launch from the scratch
    for seed, shape in ((4300, (5, 16, 8, 128, 16, 1024, 128, 300, 2048)),
                        (4400, (3, 8, 8, 128, 16, 1024, 256, 1500, 4000)),
                        (4500, (4, 32, 4, 128, 16, 1024, 256, 64, 4000))):
        case = _case(orc, torch, seed, *shape)
        need3, want3, got3 = _run_both(tmc, torch, case)
        assert need3 > 0 and not torch.isnan(want3).any()
        assert torch.equal(got3.view(torch.int16), want3.view(torch.int16))


def test_noalloc_rejects_limits_beyond_scratch(tmc):
    lib = tmc.lib()
    p = C.c_void_p(256)
    # 64 requests x 32 query heads x 64 splits of 1024 positions: 68 MB of partials
    need = tmc.attention_workspace_bytes(64, 32, 8, 128, 16 * 4096)
    assert need > lib.tmc_attention_scratch_bytes()
    assert lib.tmc_paged_decode_attention_noalloc(p, p, p, p, p, p, p, 0, 64, 32, 8, 128, 16,
                                                  4096, 8192, 8 * 16 * 128, 16 * 128, None) != 0
    assert "static scratch" in tmc.last_error()
