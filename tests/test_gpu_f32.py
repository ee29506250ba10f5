"""GPU parity of the f32 route: dmc_matmul_f32_gpu (host pointers) and
dmc_hip_gemv_f32_rd (device pointers) against the f32 oracle (the reference's
f32 `@` chain, compiler/src/jit.rs:29448-29466 and jit.rs:20715-20802), with
tests/parity.py's rule: NaN/inf classes exact, zeros bitwise, normwise 1e-5.
"""
import numpy as np
import pytest

import oracle
from parity import check, check_bound

pytestmark = pytest.mark.gpu


def edge(a, rng, frac=0.01):
    """Sprinkle subnormals, signed zeros, +-1e-38 and a few inf/NaN into a."""
    flat = a.reshape(-1)
    if flat.size == 0:
        return a
    pos = rng.integers(0, flat.size, size=max(1, int(flat.size * frac)))
    flat[pos] = rng.choice(np.array([0.0, -0.0, 1e-38, -1e-38, 1e-45, -3e-42], np.float32), size=pos.size)
    if flat.size >= 64:
        pos = rng.integers(0, flat.size, size=3)
        flat[pos] = np.array([np.inf, -np.inf, np.nan], np.float32)
    return a


def operands(m, k, n, seed, special=False):
    rng = np.random.default_rng(seed)
    l = rng.standard_normal((m, k)).astype(np.float32)
    r = rng.standard_normal((k, n)).astype(np.float32)
    if special:
        edge(l, rng)
        edge(r, rng)
    return l, r


# W @ x: l is the weight [m, k], n activation columns.  Streaming (k % 4 == 0,
# k <= 16384: 1, 3 and 7 vectors per lane) and general (odd k, k > 16384).
W_AT_X = [(4096, 4096, 1), (1000, 1000, 1), (777, 1001, 1), (300, 16384, 1), (50, 20000, 1), (64, 4, 1),
          (5, 3, 1), (3000, 6144, 1), (4096, 14336, 1), (2048, 4096, 2), (999, 4096, 3), (1500, 2000, 4),
          (513, 4097, 8), (700, 1024, 16)]


@pytest.mark.parametrize("m,k,n", W_AT_X)
def test_w_at_x_matches_the_oracle(hip, m, k, n):
    l, r = operands(m, k, n, seed=m + k + n, special=True)
    check(hip.matmul_f32_gpu(l, r), oracle.matmul_f32(l, r), what=f"f32 W@x m={m} k={k} n={n}")


# x @ W: r is the weight [k, n], m activation rows (transposed on the device).
X_AT_W = [(1, 4096, 1024), (1, 1001, 333), (2, 4096, 4096), (5, 2048, 1500), (16, 1000, 64), (1, 14336, 4096)]


@pytest.mark.parametrize("m,k,n", X_AT_W)
def test_x_at_w_matches_the_oracle(hip, m, k, n):
    l, r = operands(m, k, n, seed=7 * m + k + n, special=True)
    check(hip.matmul_f32_gpu(l, r), oracle.matmul_f32(l, r), what=f"f32 x@W m={m} k={k} n={n}")


@pytest.mark.parametrize("m,k,n", [(1024, 4096, 1), (333, 1001, 1), (1, 4096, 512), (4, 2000, 300)])
def test_within_the_rigorous_bound(hip, m, k, n):
    l, r = operands(m, k, n, seed=11)
    y = hip.matmul_f32_gpu(l, r)
    y_ref = oracle.matmul_f32(l, r)
    if n <= m:  # W @ x: output (i, j) is l row i against r column j
        for j in range(n):
            check_bound(y[:, j], y_ref[:, j], r[:, j], l, what=f"f32 bound W@x col {j}")
    else:
        for i in range(m):
            check_bound(y[i], y_ref[i], l[i], np.ascontiguousarray(r.T), what=f"f32 bound x@W row {i}")


@pytest.mark.parametrize("k", [64, 4096, 4097, 14336])
def test_zero_outputs_follow_the_reference_chain(hip, k):
    """Rows whose products all underflow: negative ones end at -0 in the
    chain, positive at +0, a sign flip at the last product takes its sign,
    exact zeros and an all-zero row give +0 -- the split sums must agree bit
    for bit (the zero rule)."""
    x = np.full(k, np.float32(1e-30), np.float32)
    w = np.full((6, k), np.float32(1e-30), np.float32)
    w[1] = -w[1]
    w[2, k - 1] = -w[2, k - 1]
    w[3] = 0
    h = k // 2
    w[4, :h] = 1.0
    w[4, h:2 * h] = -1.0
    w[4, 2 * h:] = 0.0
    x2 = np.full(k, np.float32(0.5), np.float32)
    w[5, ::2] = -w[5, ::2]
    for xv in (x, x2):
        y = hip.matmul_f32_gpu(w, xv)[:, 0]
        y_ref = oracle.matmul_f32(w, xv)[:, 0]
        z = y_ref == 0
        assert z[3] and (z[4] or xv is x), y_ref  # x2: row 4 cancels exactly
        assert np.array_equal(y[z].view(np.uint32), y_ref[z].view(np.uint32)), (y, y_ref)
        # constant-valued products: the chain's own rounding error exceeds
        # the normwise tolerance, so the nonzero rows take the rigorous bound
        check_bound(y, y_ref, xv, w, what=f"f32 zero signs k={k}")


def test_all_zero_activation_gives_positive_zero(hip):
    w = np.random.default_rng(0).standard_normal((512, 4096)).astype(np.float32)
    y = hip.matmul_f32_gpu(w, -np.zeros(4096, np.float32))
    assert np.all(y == 0) and not np.any(np.signbit(y))


def test_k_zero_writes_positive_zero(hip):
    y = hip.matmul_f32_gpu(np.zeros((8, 0), np.float32), np.zeros((0, 1), np.float32))
    assert y.shape == (8, 1) and np.all(y == 0) and not np.any(np.signbit(y))


def test_gemm_shape_is_refused_and_out_untouched(hip):
    rc, out = hip.matmul_f32_gpu_try(np.ones((17, 8), np.float32), np.ones((8, 17), np.float32))
    assert rc == -2 and np.all(out == 0)


def test_unregistered_operand_updated_in_place_is_seen(hip):
    """The reference's f32 `@` keeps nothing between calls, so an operand
    that the program updates in place -- here one element that the sampled
    content key does not read (word 1 of the buffer; the samples start at
    words 0, q, 2q, ...) -- must give the new result, in both layouts, and no
    unregistered operand may stay resident."""
    rng = np.random.default_rng(5)
    count = hip.resident_count()
    w = rng.standard_normal((2048, 4096)).astype(np.float32)      # W @ x: l is the weight
    x = rng.standard_normal(4096).astype(np.float32)
    hip.matmul_f32_gpu(w, x)
    w[0, 3] = 1.0e4
    y = hip.matmul_f32_gpu(w, x)
    check(y, oracle.matmul_f32(w, x), what="f32 W@x after an in-place update")
    a = rng.standard_normal((2, 4096)).astype(np.float32)         # x @ W: r is the weight
    r = rng.standard_normal((4096, 1024)).astype(np.float32)
    hip.matmul_f32_gpu(a, r)
    r[0, 3] = -1.0e4
    y = hip.matmul_f32_gpu(a, r)
    check(y, oracle.matmul_f32(a, r), what="f32 x@W after an in-place update")
    assert hip.resident_count() == count


def test_registered_weight_stays_resident(hip):
    """Bytes registered at an address stay resident for the f32 route (the
    caller's promise that they do not change): no new entry on W @ x, one
    transposed copy for x @ W, built once; another address with the same
    bytes is staged per call."""
    rng = np.random.default_rng(6)
    w = rng.standard_normal((2048, 4096)).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    hip.register_weight(w)
    count = hip.resident_count()
    for _ in range(2):
        y = hip.matmul_f32_gpu(w, x)
        check(y, oracle.matmul_f32(w, x), what="f32 registered W@x")
    assert hip.resident_count() == count
    r = rng.standard_normal((4096, 1024)).astype(np.float32)
    a = rng.standard_normal((3, 4096)).astype(np.float32)
    hip.register_weight(r)
    count = hip.resident_count()
    for _ in range(2):
        y = hip.matmul_f32_gpu(a, r)
        check(y, oracle.matmul_f32(a, r), what="f32 registered x@W")
    assert hip.resident_count() == count + 1
    r2 = r.copy()  # same bytes, another address: not registered
    y = hip.matmul_f32_gpu(a, r2)
    check(y, oracle.matmul_f32(a, r2), what="f32 copy of a registered weight")
    assert hip.resident_count() == count + 1


@pytest.mark.parametrize("m,k,n,stream", [(1, 4096, 14336, True), (4, 4096, 1000, True), (3, 14336, 4096, True),
                                          (1, 4097, 1000, False), (16, 102, 33, False)])
def test_device_pointer_entry(hip, m, k, n, stream):
    rng = np.random.default_rng(m * k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(w) as dw, \
            hip.DeviceBuffer(4 * m * n) as dy:
        pl = hip.plan_f32(m, k, n, x_addr=dx.addr, w_addr=dw.addr)
        assert (pl.kvec > 0) == stream, pl
        hip.gemv_f32_rd(dx, dw, dy, m, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (m, n))
    check(y, oracle.matmul_f32(x, np.ascontiguousarray(w.T)), what=f"f32 device m={m} k={k} n={n}")


@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
def test_full_decode_shapes_on_sampled_rows(hip, n, k):
    """C2-sized f32 weights (235 MB) on the device, W @ x through the drop-in;
    every row of the result against the closed form on a sample of rows plus
    the first and last rows of each 1024-row block."""
    rng = np.random.default_rng(n)
    w = (np.float32(0.02) * rng.standard_normal((n, k), dtype=np.float32))
    x = rng.standard_normal(k, dtype=np.float32)
    y = hip.matmul_f32_gpu(w, x)[:, 0]
    rows = np.unique(np.concatenate([rng.integers(0, n, 256), np.arange(0, n, 1024), np.arange(1023, n, 1024)]))
    y_ref = oracle.gemv_points_f32(x, w, np.zeros(rows.size, np.int64), rows)
    check(y[rows], y_ref, what=f"f32 full W[{n},{k}] sampled")
    assert np.all(np.isfinite(y))


X14_F32 = [(4096, 14336), (4097, 14336), (1030, 12288), (6, 9000), (300, 4100)]


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", X14_F32)
def test_fourteen_waves_f32(hip, n, k, m, monkeypatch):
    """The 14-wave kernel with f32 weights (the default where the 8-wave
    kernel would take the activation rows in several passes;
    DMC_HIP_F32_X14=2 takes it wherever it applies): 2 to 4 windows of 4
    weights per lane, a partial last workgroup (n = 4097), fewer rows than one
    workgroup (n = 6), edge values; through the device-pointer entry (y [m,n])
    and the drop-in's W @ x (out [n,m]: the other output orientation); two
    launches bit for bit alike."""
    monkeypatch.setenv("DMC_HIP_F32_X14", "2")
    rng = np.random.default_rng(n + k + m)
    x = edge(rng.standard_normal((m, k)).astype(np.float32), rng)
    w = edge(rng.standard_normal((n, k)).astype(np.float32), rng)
    y_ref = oracle.matmul_f32(x, np.ascontiguousarray(w.T))
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(w) as dw, \
            hip.DeviceBuffer(4 * m * n) as dy:
        pl = hip.plan_f32(m, k, n, x_addr=dx.addr, w_addr=dw.addr)
        assert (pl.waves, pl.mt, pl.rows_per_group) == (14, m, 16), pl
        ys = []
        for _ in range(2):
            hip.gemv_f32_rd(dx, dw, dy, m, k, n)
            hip.synchronize()
            ys.append(dy.download(np.float32, (m, n)))
    assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))
    check(ys[0], y_ref, what=f"f32 x14 device m={m} n={n} k={k}")
    check(hip.matmul_f32_gpu(w, np.ascontiguousarray(x.T)), np.ascontiguousarray(y_ref.T),
          what=f"f32 x14 W@x m={m} n={n} k={k}")


X8_F32 = [(14336, 4096), (4097, 4096), (1030, 3000), (6, 2052), (300, 4096), (1792, 3072)]


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", X8_F32)
def test_eight_wave_group_f32(hip, n, k, m, monkeypatch):
    """The f32 weights' 8-wave group (2048 < K <= 4096, two windows of 4
    weights per lane; the default at 3 and 4 activation rows and where K is
    not a multiple of 2048, DMC_HIP_F32_X8=2 here): a partial last workgroup
    (n = 4097), lanes past K (k = 3000, 2052), fewer rows than one workgroup
    (n = 6), edge values; through the device-pointer entry and the drop-in's
    W @ x; two launches bit for bit alike."""
    monkeypatch.setenv("DMC_HIP_F32_X8", "2")
    rng = np.random.default_rng(3 * n + k + m)
    x = edge(rng.standard_normal((m, k)).astype(np.float32), rng)
    w = edge(rng.standard_normal((n, k)).astype(np.float32), rng)
    y_ref = oracle.matmul_f32(x, np.ascontiguousarray(w.T))
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(w) as dw, \
            hip.DeviceBuffer(4 * m * n) as dy:
        pl = hip.plan_f32(m, k, n, x_addr=dx.addr, w_addr=dw.addr)
        assert (pl.waves, pl.kvec, pl.mt, pl.rows_per_group, pl.grid_x) == (8, 2, m, 16, -(-n // 16)), pl
        ys = []
        for _ in range(2):
            hip.gemv_f32_rd(dx, dw, dy, m, k, n)
            hip.synchronize()
            ys.append(dy.download(np.float32, (m, n)))
    assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))
    check(ys[0], y_ref, what=f"f32 x8 device m={m} n={n} k={k}")
    check(hip.matmul_f32_gpu(w, np.ascontiguousarray(x.T)), np.ascontiguousarray(y_ref.T),
          what=f"f32 x8 W@x m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [3, 4])
def test_eight_wave_group_f32_zero_rule(hip, m):
    """Exact zeros on the f32 8-wave group at its default shapes (K = 4096,
    3 or 4 activation rows): the patterns of the 14-wave test, bit for bit
    the reference."""
    k, n = 4096, 4096
    x = np.full((m, k), np.float32(1e-30), np.float32)
    x[1::2] = np.float32(0.5)
    w = np.full((n, k), np.float32(1e-30), np.float32)
    w[1::6] = -w[1::6]
    w[2::6, k - 1] = -w[2::6, k - 1]
    w[3::6] = 0
    h = k // 2
    w[4::6, :h] = 1.0
    w[4::6, h:] = -1.0
    w[5::6, ::2] = -w[5::6, ::2]
    pl = hip.plan_f32(m, k, n, x_addr=256, w_addr=256)
    assert (pl.waves, pl.rows_per_group) == (8, 16), pl
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(w) as dw, \
            hip.DeviceBuffer(4 * m * n) as dy:
        hip.gemv_f32_rd(dx, dw, dy, m, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (m, n))
    rows = np.r_[0:12, n - 12:n]
    y_ref = oracle.matmul_f32(x, np.ascontiguousarray(w[rows].T))
    z = y_ref == 0
    assert np.any(z)
    assert np.array_equal(y[:, rows][z].view(np.uint32), y_ref[z].view(np.uint32)), (y[:, rows], y_ref)
    for r in range(m):
        check_bound(y[r, rows], y_ref[r], x[r], w[rows], what=f"f32 x8 zero rule m={m} row {r}")


@pytest.mark.parametrize("m", [2, 4])
def test_fourteen_waves_f32_zero_rule(hip, m, monkeypatch):
    """Exact zeros on the f32 14-wave kernel (the default at K = 14336 and
    2 or more activation rows over 4096 rows): products that all underflow
    (-0 / +0 by their sign in the chain), a sign flip at the last product,
    exact-zero rows, an exact cancellation -- bit for bit the reference."""
    k, n = 14336, 4096
    rng = np.random.default_rng(m)
    x = np.full((m, k), np.float32(1e-30), np.float32)
    x[1::2] = np.float32(0.5)
    w = np.full((n, k), np.float32(1e-30), np.float32)
    w[1::6] = -w[1::6]
    w[2::6, k - 1] = -w[2::6, k - 1]
    w[3::6] = 0
    h = k // 2
    w[4::6, :h] = 1.0
    w[4::6, h:] = -1.0
    w[5::6, ::2] = -w[5::6, ::2]
    assert hip.plan_f32(m, k, n, x_addr=256, w_addr=256).waves == 14
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(w) as dw, \
            hip.DeviceBuffer(4 * m * n) as dy:
        hip.gemv_f32_rd(dx, dw, dy, m, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (m, n))
    rows = np.r_[0:12, n - 12:n]
    y_ref = oracle.matmul_f32(x, np.ascontiguousarray(w[rows].T))
    z = y_ref == 0
    assert np.any(z)
    assert np.array_equal(y[:, rows][z].view(np.uint32), y_ref[z].view(np.uint32)), (y[:, rows], y_ref)
    for r in range(m):
        check_bound(y[r, rows], y_ref[r], x[r], w[rows], what=f"f32 x14 zero rule m={m} row {r}")
