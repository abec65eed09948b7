"""GPU: a preempted request's KV pages spill raw into pinned host memory and
come back bit for bit into other pages (the serving layer's preemption path,
ServingRuntime.cpp:426-930 semantics: snapshot, release, resume)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 16


@pytest.fixture(scope="module")
def rt(host, tmc):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    runtime = host.HipRuntime()
    assert runtime.is_available(), runtime.initialization_error()
    return runtime


def _plan(host, heads=4, d=128, capacity=256):
    plan = host.KVCachePlan()
    plan.heads, plan.head_dimension, plan.capacity = heads, d, capacity
    plan.dtype = host.DType.Float16
    return plan


def _fill(tmc, pointer, count, seed):
    lib = tmc.lib()
    rc = lib.tmc_fill_normal(C.c_void_p(pointer), 0, count, seed, 0.0, 1.0, None)
    assert rc == 0, lib.tmc_last_error()


def test_spill_and_restore_pages_bit_exact(host, tmc, rt):
    plan = _plan(host)
    pool = host.create_kv_page_pool(rt, plan, P, 32)
    count = pool.capacity_pages() * pool.page_elements()
    _fill(tmc, pool.key_pointer(), count, 11)
    _fill(tmc, pool.value_pointer(), count, 12)
    assert rt.synchronize() == ""
    state = host.create_kv_cache_state(rt, plan, pool, False)
    assert state.stage_length(rt, 40) == ""
    state.commit_length(40)
    keys, values = state.read_key_prefix(), state.read_value_prefix()
    before = state.page_table()
    spill = state.spill_pages(rt)
    assert spill.length == 40 and spill.pages == 3
    assert spill.page_bytes == 4 * P * 128 * 2 and spill.bytes() == 2 * 3 * spill.page_bytes
    assert state.reset(rt) == "" and pool.used_pages() == 0
    # another request takes the released pages and the pool is overwritten
    other = host.create_kv_cache_state(rt, plan, pool, False)
    assert other.stage_length(rt, 20) == ""
    _fill(tmc, pool.key_pointer(), count, 13)
    _fill(tmc, pool.value_pointer(), count, 14)
    assert rt.synchronize() == ""
    assert state.restore_pages(rt, spill) == ""
    assert state.current_length() == 40
    after = state.page_table()
    assert len(after) == 3 and not set(after) & set(other.page_table()) and after != before
    np.testing.assert_array_equal(state.read_key_prefix(), keys)
    np.testing.assert_array_equal(state.read_value_prefix(), values)
    # a restore needs an empty state and a matching spill
    assert "empty" in state.restore_pages(rt, spill)
    small = host.create_kv_cache_state(rt, _plan(host, heads=2), host.create_kv_page_pool(
        rt, _plan(host, heads=2), P, 16), False)
    assert "does not match" in small.restore_pages(rt, spill)


def test_spill_requires_device_pages(host, rt):
    plan = _plan(host)
    pool = host.create_host_kv_page_pool(plan, P, 16)
    state = host.create_kv_cache_state(rt, plan, pool, False)
    assert state.stage_length(rt, 5) == ""
    state.commit_length(5)
    with pytest.raises(RuntimeError, match="paged device storage"):
        state.spill_pages(rt)
