"""GPU: the error-returning drop-in forms and the resident-weight policy.

The try forms (include/dmc_hip.h) take the drop-in entries' arguments and
return DMC_HIP_E* instead of aborting, leaving `out` untouched, so a JIT can
fall back to its own CPU kernel as the reference does (gpu.rs:327-332,
gpu.rs:483-486).  DMC_HIP_RESIDENT_CAP caps resident weight bytes, which
forces the out-of-memory path without exhausting the device.
"""
import numpy as np
import pytest

import oracle
from demonic_amd import _lib
from demonic_amd import workloads as W
from parity import check

pytestmark = pytest.mark.gpu

ENOMEM = -3


def data(m, k, n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = W.bf16_rne(np.float32(0.02) * rng.standard_normal((n, k)).astype(np.float32))
    return x, w


def test_try_forms_match_the_void_forms(hip):
    lib = _lib.load()
    x, w = data(3, 1000, 700, seed=1)
    wt = np.ascontiguousarray(w.T)
    m, k, n = 3, 1000, 700
    out = np.full((m, n), np.nan, np.float32)
    assert lib.dmc_matmul_bf16_gpu_t_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, m, k, n) == 0
    assert np.array_equal(out.view(np.uint32), hip.matmul_bf16_gpu_t(x, w).view(np.uint32))
    out[:] = np.nan
    assert lib.dmc_matmul_bf16_gpu_try(x.ctypes.data, wt.ctypes.data, out.ctypes.data, m, k, n) == 0
    assert np.array_equal(out.view(np.uint32), hip.matmul_bf16_gpu(x, wt).view(np.uint32))
    check(out, oracle.matmul_bf16_t(x, w), what="try x @ W")
    # batched: two slices, x broadcast (ls = 0)
    xb = np.ascontiguousarray(x[0])
    wb = np.concatenate([wt.reshape(-1), wt.reshape(-1)[::-1].copy()])
    ob = np.full(2 * n, np.nan, np.float32)
    assert lib.dmc_matmul_bf16_gpu_batched_try(xb.ctypes.data, wb.ctypes.data, ob.ctypes.data, 1, k, n, 2, 0,
                                               k * n) == 0
    want = hip.matmul_bf16_gpu_batched(xb, wb, 1, k, n, 2, 0, k * n)
    assert np.array_equal(ob.view(np.uint32), want.view(np.uint32))
    # deferred: written by the flush
    od = np.full(2 * n, np.nan, np.float32)
    assert lib.dmc_matmul_bf16_gpu_batched_deferred_try(xb.ctypes.data, wb.ctypes.data, od.ctypes.data, 1, k, n,
                                                        2, 0, k * n) == 0
    assert lib.dmc_matmul_bf16_gpu_flush_try() == 0
    assert np.array_equal(od.view(np.uint32), want.view(np.uint32))


def test_out_of_memory_returns_enomem_and_leaves_out_untouched(hip, monkeypatch):
    """With resident weights capped below the weight's size, every try form
    returns DMC_HIP_ENOMEM, writes nothing and queues nothing; without the
    cap the same call succeeds."""
    lib = _lib.load()
    hip.release_weights()
    m, k, n = 1, 1024, 2048                       # a 4 MiB weight
    x, w = data(m, k, n, seed=2)
    wt = np.ascontiguousarray(w.T)
    monkeypatch.setenv("DMC_HIP_RESIDENT_CAP", str(1 << 20))
    out = np.full(n, 7.0, np.float32)
    p = (x.ctypes.data, wt.ctypes.data, out.ctypes.data)
    assert lib.dmc_matmul_bf16_gpu_try(*p, m, k, n) == ENOMEM
    assert lib.dmc_matmul_bf16_gpu_t_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, m, k, n) == ENOMEM
    assert lib.dmc_matmul_bf16_gpu_batched_try(*p, m, k, n, 1, 0, 0) == ENOMEM
    assert lib.dmc_matmul_bf16_gpu_batched_deferred_try(*p, m, k, n, 1, 0, 0) == ENOMEM
    assert b"device memory" in lib.dmc_hip_last_error()
    assert lib.dmc_matmul_bf16_gpu_flush_try() == 0  # nothing was queued
    assert np.all(out == 7.0)
    assert hip.resident_count() == 0
    monkeypatch.delenv("DMC_HIP_RESIDENT_CAP")
    assert lib.dmc_matmul_bf16_gpu_try(*p, m, k, n) == 0
    check(out[None], oracle.matmul_bf16_t(x, w), what="after the cap is lifted")


def test_registered_weight_survives_evictions(hip, monkeypatch):
    """dmc_hip_register_weight hands out a device address, so its entry is
    pinned: the resident cap and the cached-entry evictions it triggers never
    free it.  Drop-in calls on other weights churn the cache under a byte cap,
    then the registered address still computes the right GEMV on the device."""
    hip.release_weights()
    m, k, n = 1, 2048, 1024                       # 4 MiB each
    x, w = data(m, k, n, seed=3)
    addr = hip.register_weight(w)
    assert addr and hip.resident_count() == 1
    monkeypatch.setenv("DMC_HIP_RESIDENT_CAP", str(10 << 20))  # room for the pinned weight and one more
    for s in range(4):
        xo, wo = data(m, k, n, seed=100 + s)
        y = hip.matmul_bf16_gpu_t(xo, wo)
        check(y, oracle.matmul_bf16_t(xo, wo), what=f"churn {s}")
        assert hip.resident_count() <= 2
    assert hip.register_weight(w) == addr          # still resident, same address
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer(4 * n) as dy:
        _lib.check(_lib.load().dmc_hip_gemv_rd(dx.addr, addr, dy.addr, m, k, n))
        hip.synchronize()
        check(dy.download(np.float32, (m, n)), oracle.matmul_bf16_t(x, w), what="registered after churn")
    monkeypatch.delenv("DMC_HIP_RESIDENT_CAP")
    hip.release_weights()
    assert hip.resident_count() == 0 and hip.resident_bytes() == 0


def test_consecutive_calls_see_each_new_x(hip):
    """Back-to-back synchronous calls on one resident weight, each with a new
    activation written into the same staging slice: every result is the
    oracle's for that call's x (no stale activation survives from the call
    before, whichever way x reaches the kernels)."""
    m, k, n = 1, 4096, 1536
    _, w = data(m, k, n, seed=5)
    wt = np.ascontiguousarray(w.T)
    rng = np.random.default_rng(6)
    xs = [rng.standard_normal((m, k)).astype(np.float32) for _ in range(3)]
    want = [oracle.matmul_bf16_t(x, w) for x in xs]
    for i in range(12):
        y = hip.matmul_bf16_gpu_t(xs[i % 3], w)
        assert np.array_equal(y.view(np.uint32), hip.matmul_bf16_gpu(xs[i % 3], wt).view(np.uint32)), i
        check(y, want[i % 3], what=f"call {i}")


def test_calls_from_several_threads(hip):
    """One process-wide context, its entries serialized by a mutex (the
    reference keeps one context per thread, gpu.rs:186-189): four threads
    issue synchronous bf16 and f32 calls on their own weights and
    activations, interleaved; every result is its own call's."""
    import threading

    cases = []
    for t in range(4):
        x, w = data(1 + t % 2, 1024 + 8 * t, 300 + 17 * t, seed=700 + t)
        wf = np.random.default_rng(800 + t).standard_normal((64 + t, 512)).astype(np.float32)
        xf = np.random.default_rng(900 + t).standard_normal(512).astype(np.float32)
        cases.append((x, w, oracle.matmul_bf16_t(x, w), wf, xf, oracle.matmul_f32(wf, xf)))
    errors = []

    def worker(t):
        x, w, ref, wf, xf, ref_f = cases[t]
        try:
            for i in range(25):
                if (i + t) % 3:
                    check(hip.matmul_bf16_gpu_t(x, w), ref, what=f"thread {t} call {i}")
                else:
                    check(hip.matmul_f32_gpu(wf, xf), ref_f, what=f"thread {t} f32 call {i}")
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert not errors, errors[:2]
