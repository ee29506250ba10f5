"""GPU: dmc_hip_gemv_cs_noalloc, the column-stream GEMV that allocates
nothing (its split-k partial sums live in a fixed 32 MiB device array).

It must give dmc_hip_gemv_cs's results bit for bit -- the same kernels, a
different home for the partials -- on consecutive calls, a smaller one after
a larger one (the array keeps the first call's partials), and reject a shape
whose partials do not fit.
"""
import numpy as np
import pytest

import oracle
from demonic_amd import _lib
from demonic_amd import workloads as W
from parity import check

pytestmark = pytest.mark.gpu

EINVAL = -2
LIMIT = 32 << 20


def run(hip, entry, x, wt, m, k, n, batch, ls, rs):
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(wt) as dw, \
            hip.DeviceBuffer(4 * batch * m * n) as dy:
        dy.upload(np.full(batch * m * n, np.nan, np.float32))
        _lib.check(entry(dx.addr, dw.addr, dy.addr, m, k, n, batch, ls, rs))
        hip.synchronize()
        return dy.download(np.float32, (batch * m * n,))


@pytest.mark.parametrize("shapes", [[(2, 4096, 14336, 1), (1, 1000, 515, 3)]])
def test_noalloc_matches_gemv_cs_on_consecutive_calls(hip, shapes):
    lib = _lib.load()
    assert hip.available()
    for m, k, n, batch in shapes:   # the second call is smaller, with odd N (the unaligned kernel)
        p = hip.plan("cs", m, k, n, batch=batch, rs=k * n)
        assert 0 < p.workspace_bytes <= LIMIT, p   # the split-k partials do use the scratch
        rng = np.random.default_rng(m * 1000 + n)
        x = rng.standard_normal(batch * m * k).astype(np.float32)
        wt = W.bf16_rne(np.float32(0.02) * rng.standard_normal(batch * k * n).astype(np.float32))
        want = run(hip, lib.dmc_hip_gemv_cs, x, wt, m, k, n, batch, m * k, k * n)
        got = run(hip, lib.dmc_hip_gemv_cs_noalloc, x, wt, m, k, n, batch, m * k, k * n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (m, k, n, batch)
        for z in range(batch):
            xz = x[z * m * k:(z + 1) * m * k].reshape(m, k)
            wz = wt[z * k * n:(z + 1) * k * n].reshape(k, n)
            check(got[z * m * n:(z + 1) * m * n].reshape(m, n), oracle.matmul_bf16(xz, wz),
                  what=f"noalloc m={m} k={k} n={n} slice {z}")


def test_noalloc_rejects_partials_beyond_the_fixed_scratch(hip):
    """Odd N always sums slices in a second pass; 512 slices of 4 x 4097
    outputs need 33,562,624 bytes of partials, 8 KiB beyond the array: the
    call returns DMC_HIP_EINVAL before launching anything."""
    lib = _lib.load()
    m, k, n, batch = 4, 64, 4097, 512
    p = hip.plan("cs", m, k, n, batch=batch, rs=k * n)
    assert p.workspace_bytes > LIMIT, p
    x = np.zeros(batch * m * k, np.float32)
    wt = np.zeros(batch * k * n, np.uint16)
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(wt) as dw, \
            hip.DeviceBuffer(4 * batch * m * n) as dy:
        dy.upload(np.full(batch * m * n, 5.0, np.float32))
        rc = lib.dmc_hip_gemv_cs_noalloc(dx.addr, dw.addr, dy.addr, m, k, n, batch, m * k, k * n)
        assert rc == EINVAL, rc
        assert b"fixed maximum" in lib.dmc_hip_last_error()
        hip.synchronize()
        assert np.all(dy.download(np.float32, (batch * m * n,)) == 5.0)
