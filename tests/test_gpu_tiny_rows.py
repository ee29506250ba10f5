"""MFMA layouts on activation rows whose every entry is tiny.

The MFMA kernels take x as three bf16 terms, exact only for |x| >= 2^-110
(below that the last term falls under bf16's least subnormal, 2^-133).  A
row whose largest |x| over a workgroup's k range is nonzero and below 2^-100
therefore takes the reference chain over that range instead of its MFMA sums
(gemv_kernels.hip, "Tiny activation rows").  Here rows of N(0,1) * 1e-36 and
N(0,1) * 1e-37 against N(0, 0.02) weights -- products near 2e-38 (normal)
and 2e-39 (subnormal in f32) -- sit beside ordinary rows and an all-zero row,
on each forced MFMA layout (wide 6, rows16 7, gemm 8: x split in the kernel
or by a launch into planes), with k in one slice and split over several.
Every activation row is held to the 1e-5 normwise rule on its own (an
ordinary row beside it would otherwise hide a tiny row's error), and where
k is not split a tiny row's outputs equal the oracle bit for bit (they are
the reference chain).  C4's own plans at M = 4, 8, 16 on the full LM head
are in tests/test_gpu_configs.py.
"""
import numpy as np
import pytest

import oracle
from demonic_amd import workloads as W
from parity import check

SCALES = (np.float32(1e-36), np.float32(1e-37))


def tiny_rows_x(m, k, seed):
    """x [m,k]: rows 0, 3, 6, ... at 1e-36, rows 1, 4, 7, ... at 1e-37, the
    others ordinary N(0,1); the last row all zeros when m > 3."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    for r in range(m):
        if r % 3 < 2:
            x[r] *= SCALES[r % 3]
    if m > 3:
        x[-1] = 0.0
    return x


def tiny_set(m):
    return [r for r in range(m) if r % 3 < 2 and not (m > 3 and r == m - 1)]


def check_rows(y, y_ref, m, what, exact):
    for r in range(m):
        check(y[r], y_ref[r], what=f"{what} row {r}")
    if exact:
        for r in tiny_set(m):
            assert np.array_equal(y[r].view(np.uint32), y_ref[r].view(np.uint32)), \
                f"{what}: tiny row {r} is not the reference chain"


def run(hip, x, w, m, k, n):
    with hip.DeviceBuffer.from_numpy(w) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * m * n) as dy:
        p = hip.plan("rd", m, k, n, x_addr=dx.addr, w_addr=dw.addr)
        dy.upload(np.full(m * n, np.nan, np.float32))
        hip.gemv_rd(dx, dw, dy, m, k, n)
        hip.synchronize()
        return p, dy.download(np.float32, (m, n))


# (kind, m, k, n, extra env): k split where the plan's workspace is nonzero
CASES = [
    (6, 16, 4096, 1000, {}), (6, 5, 1024, 300, {}),
    (7, 4, 4096, 1000, {}), (7, 8, 4096, 1000, {}), (7, 16, 4096, 1000, {}), (7, 3, 64, 40, {}),
    (7, 4, 14336, 4096, {}), (7, 12, 14336, 4096, {}),                 # k in 2 and 4 slices
    (8, 16, 4096, 1000, {"DMC_HIP_GEMM_FUSE": "2"}), (8, 16, 4096, 1000, {"DMC_HIP_GEMM_FUSE": "0"}),
    (8, 16, 14336, 4096, {}),                                          # k slices, x split in the kernel
    (8, 40, 4096, 1000, {}), (8, 24, 14336, 4096, {"DMC_HIP_GEMM_FUSE": "0"}),
]


@pytest.mark.gpu
@pytest.mark.parametrize("kind,m,k,n,env", CASES)
def test_tiny_activation_rows(hip, kind, m, k, n, env, monkeypatch):
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", str(kind))
    for key, v in env.items():
        monkeypatch.setenv(key, v)
    rng = np.random.default_rng(m * 131 + k + n + kind)
    w = W.bf16_rne(np.float32(0.02) * rng.standard_normal((n, k), dtype=np.float32))
    x = tiny_rows_x(m, k, seed=kind * 1000 + m)
    p, y = run(hip, x, w, m, k, n)
    assert p.slices == -kind, p
    rows = np.unique(np.r_[0, n - 1, rng.integers(0, n, 200)]) if n * k > (1 << 22) else np.arange(n)
    mi, ni = np.meshgrid(np.arange(m), rows, indexing="ij")
    y_ref = oracle.gemv_points(x, w, "rd", mi.reshape(-1), ni.reshape(-1)).reshape(m, -1)
    check_rows(y[:, rows], y_ref, m, f"tiny rows kind={kind} m={m} k={k} n={n} {env}",
               exact=p.workspace_bytes == 0 or kind == 6)
    if m > 3:  # the all-zero row: +0 everywhere
        assert np.all(y[-1] == 0) and not np.any(np.signbit(y[-1]))


def test_tiny_rows_before_the_fix_would_fail():
    """The size of the hole on the CPU: x split into three truncated bf16
    terms loses, for a row at 1e-37, far more than the 1e-5 rule allows --
    so the GPU cases above test the fix, not a tolerance."""
    rng = np.random.default_rng(1)
    k = 4096
    w = W.bf16_to_f32(W.bf16_rne(np.float32(0.02) * rng.standard_normal((64, k), dtype=np.float32)))
    x = (rng.standard_normal(k).astype(np.float32) * SCALES[1]).astype(np.float32)

    def trunc(v):
        return (v.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)

    def bf16_sub(v):  # bf16 keeps nothing below 2^-133
        q = np.float32(2.0 ** -133)
        return (np.trunc(v / q) * q).astype(np.float32)

    hi = trunc(x)
    mid = bf16_sub(trunc((x - hi).astype(np.float32)))
    lo = bf16_sub(trunc((x - hi - mid).astype(np.float32)))
    split = hi.astype(np.float64) + mid + lo
    exact = w.astype(np.float64) @ x.astype(np.float64)
    approx = w.astype(np.float64) @ split
    assert np.linalg.norm(approx - exact) / np.linalg.norm(exact) > 1e-4
