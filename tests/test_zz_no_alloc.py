"""The allocation-free decode GEMM (catena_mi355x_gemm_bf16_decode_noalloc)
against catena_mi355x_gemm_bf16, through the C ABI: the same bits on two
calls in a row (the second smaller, so it runs on the scratch the first
left behind), no device allocation by the call, and the size limit."""
import ctypes

import numpy as np
import pytest

import catena_amd as ca
from gpu_util import dev_normal_bf16, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _init():
    say("init device 0")
    ca.init(0)


def _pair(m, n, k, seed):
    x = dev_normal_bf16(m * k, seed, 0, 1.0)
    w = dev_normal_bf16(k * n, seed, 1, 0.02)
    return x, w


def test_noalloc_decode_gemm_equals_the_allocating_entry_point():
    """shutdown + init first: that releases the split-K workspace the
    allocating entry point keeps, so a call that fell back to it would have
    to allocate.  The allocation-free calls then run before any allocating
    call, and the pool must not change across them."""
    L = ca.lib()
    say("shutdown + init (releases the library's split-K workspace)")
    ca.shutdown()
    ca.init(0)
    # two calls in a row per output type, the second with a smaller input;
    # both split K (8 and 2 k groups), so both write partials into the scratch
    shapes = [(16, 4096, 11008, 61), (5, 1024, 2048, 62)]
    cases = []
    for (m, n, k, seed) in shapes:
        groups, pbytes = ca.gemm_bf16_decode_plan(m, n, k)
        assert groups > 1 and 0 < pbytes <= 4 << 20
        x, w = _pair(m, n, k, seed)
        for out_f32, dt, es in ((False, np.uint16, 2), (True, np.uint32, 4)):
            cases.append((m, n, k, x, w, out_f32, dt, ca.Buffer(m * n * es), ca.Buffer(m * n * es)))
    ca.synchronize()
    before = ca.pool_stats()
    for (m, n, k, x, w, out_f32, dt, got, _) in cases:
        say(f"decode GEMM M={m} N={n} K={k} out_f32={out_f32}: allocation-free entry point")
        st = L.catena_mi355x_gemm_bf16_decode_noalloc(x.ptr, w.ptr, got.ptr, m, n, k,
                                                      1 if out_f32 else 0)
        assert st == 0, ca.last_error()
    ca.synchronize()
    after = ca.pool_stats()
    assert after["device_allocs"] == before["device_allocs"]
    assert after["bytes_live"] == before["bytes_live"]
    for (m, n, k, x, w, out_f32, dt, got, want) in cases:
        say(f"decode GEMM M={m} N={n} K={k} out_f32={out_f32}: allocating entry point")
        ca.gemm_bf16(x, w, want, m, n, k, out_f32=out_f32)
        ca.synchronize()
        assert np.array_equal(got.read(dt), want.read(dt)), (m, n, k, out_f32)


def test_noalloc_decode_gemm_limits():
    L = ca.lib()
    # partials of 3 k groups x 16 x 24224 f32 = 4.4 MiB: beyond the 4 MiB scratch
    groups, pbytes = ca.gemm_bf16_decode_plan(16, 24224, 2056)
    assert pbytes > 4 << 20
    x, w = _pair(16, 24224, 2056, 63)
    y = ca.Buffer(16 * 24224 * 2)
    say("allocation-free decode GEMM beyond its scratch (refused before launch)")
    st = L.catena_mi355x_gemm_bf16_decode_noalloc(x.ptr, w.ptr, y.ptr, 16, 24224, 2056, 0)
    assert st == 2 and "scratch" in ca.last_error()
    # not a decode shape
    st = L.catena_mi355x_gemm_bf16_decode_noalloc(x.ptr, w.ptr, y.ptr, 17, 128, 128, 0)
    assert st == 1
    # a shape that does not split K needs no scratch at all
    x2, w2 = _pair(8, 32000, 2048, 64)
    assert ca.gemm_bf16_decode_plan(8, 32000, 2048) == (1, 0)
    a, b = ca.Buffer(8 * 32000 * 2), ca.Buffer(8 * 32000 * 2)
    say("allocation-free decode GEMM without a k split")
    ca.gemm_bf16(x2, w2, a, 8, 32000, 2048)
    assert L.catena_mi355x_gemm_bf16_decode_noalloc(x2.ptr, w2.ptr, b.ptr, 8, 32000, 2048, 0) == 0
    assert np.array_equal(a.read(np.uint16), b.read(np.uint16))


def test_noalloc_decode_gemm_random_shapes():
    """Seeded random decode shapes within the scratch limit (split K or not,
    ragged column blocks, both output types), each called twice through the
    allocation-free entry point (the second call on the scratch the first
    left) and compared with the allocating entry point."""
    L = ca.lib()
    rng = np.random.default_rng(65)
    done = 0
    while done < 10:
        m = int(rng.integers(1, 17))
        n = 8 * int(rng.integers(1, 3000))
        k = 8 * int(rng.integers(1, 2000))
        groups, pbytes = ca.gemm_bf16_decode_plan(m, n, k)
        if pbytes > 4 << 20:
            continue
        out_f32 = bool(rng.integers(0, 2))
        dt, es = (np.uint32, 4) if out_f32 else (np.uint16, 2)
        x, w = _pair(m, n, k, 70 + done)
        got, want = ca.Buffer(m * n * es), ca.Buffer(m * n * es)
        say(f"allocation-free decode GEMM random M={m} N={n} K={k} groups={groups} out_f32={out_f32}")
        for _ in range(2):
            st = L.catena_mi355x_gemm_bf16_decode_noalloc(x.ptr, w.ptr, got.ptr, m, n, k,
                                                          1 if out_f32 else 0)
            assert st == 0, ca.last_error()
        ca.gemm_bf16(x, w, want, m, n, k, out_f32=out_f32)
        ca.synchronize()
        assert np.array_equal(got.read(dt), want.read(dt)), (m, n, k, out_f32)
        done += 1
